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
// MFMA core (every mode): a wave owns 64 query rows as two 32-query column groups and consumes
// key tiles staged in LDS with v_mfma_f32_32x32x16_bf16:
//   S^T (32 keys x 32 queries)  = K . Q^T    A = K rows from LDS, B = Q kept in registers
//   O^T (64 d    x 32 queries) += V^T . P^T  A = transposed V tile from LDS, B = P in registers
// In the S^T accumulator a lane holds one query and 16 keys of every 32, so row max / row sum
// need one cross-half exchange (v_permlane32_swap). Softmax uses base-2 exponentials against a
// lazily moved reference maximum: no per-tile maximum is taken; the reference (and O, l) move only
// when a tile's partial row sum exceeds 2^64. Row sums are dot2 products of the bf16 P values
// that feed the PV product; walks without a reference maximum (FAST) sum the same P values on the
// matrix core instead (v_mfma_f32_4x4x4_16b_bf16 against a 0/1 selector, next to the PV product).
//
// Shared mode (dense, frame-local, anchor+local, anchor, special rows of the dynamic patterns):
// a workgroup of four waves owns up to four consecutive query tiles with one key sequence. Full
// key tiles (8 KB K + 8 KB transposed V) stream through a 4-stage LDS ring filled by
// global_load_lds_dwordx4 (no register staging), two tiles per barrier; all four waves consume
// each staged tile. A wave issues its share of the next pair's loads right after the score MFMAs
// of the current tile, so the memory-pipeline stall overlaps matrix work.
// Split mode (patch rows of block-dynamic heads): a workgroup owns one query tile; its four waves
// split the tile's block list into quarters and each streams its own 32-key half tiles through a
// private 2-slot LDS ring (no barriers). Half tiles beyond a partial block's population are never
// loaded. The four partial (max, sum, O) are merged through LDS at the end.
// Phase alignment: work-groups start at scattered times, so if every one walked its key sequence
// from the start, the tiles in use at any moment would span the whole head (45 MB at 128 frames)
// and L2 (4 MB per XCD) would miss on most of them. Instead a work-group starts its walk (and wraps
// around) at the position that the device's constant-rate clock, divided by the expected time per
// step, points to: all resident work-groups then touch nearby key frames at the same moment. The
// walk order changes only the summation order; the host can turn it off for run-to-run identical
// output.
#include <type_traits>

#include "common.h"

namespace saf3r {

constexpr int kRing = 65536;     // LDS arena shared by both modes
constexpr int kStages = 4;       // shared mode: 4 x 16 KB
constexpr int kMaxList = 3968;   // compacted block list of a split-mode tile
constexpr int kMaxSegs = 2 * kMaxHeads;

enum ItemKind { kShared = 0, kSplit = 1, kSkip = 2 };

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
  uint32_t nsmagic;  // ceil(2^32 / ns): frame of a special slot = umulhi(slot, nsmagic); 0 for ns <= 1
  uint64_t phase_dense;  // default wall-clock ticks per key-tile step of a dense walk (0: fixed order)
  uint64_t phase_split;  // default wall-clock ticks per list position of a split-mode wave (0: fixed order)
  unsigned long long* pace;  // caller's pacing state [2 kinds][3 slots][ticks, steps] (may be null)
  int pace_read;             // slot measured by the previous call: its step time paces this launch
  int pace_acc;              // slot this launch's walks add their (ticks, steps) to
  int pace_zero;             // slot cleared for the next call
  const __bf16* kc;      // KEYSET heads: compact K [set][cap][64]
  const __bf16* vc;      // KEYSET heads: compact transposed V tiles [set][cap/64][64][64]
  const int32_t* ks_count;
  int64_t ks_cap;
  const __bf16* bq;      // BROADCAST heads: frame 0 Q rows [head][bcap][64]
  const __bf16* bk;      // BROADCAST heads: frame 0 K rows [head][bcap][64]
  const __bf16* bv;      // BROADCAST heads: V tiles [head][frame][bcap/64][64][64]
  int bcap;              // ceil(T/64)*64
  uint64_t tok_order;    // DENSE heads (bit h) packed in token order: tile t = tokens 64t .. 64t+63
  uint64_t framed;       // frame-relative heads (bit h) in the framed layout: frame f = tiles f*NBT ..
  uint64_t q_pre;        // heads (bit h) whose Q rows hold q * scale * log2(e)
  int n_items;           // fixup launch: items in the segments, work-groups of the launch
  int fix_groups;
  int ntok;              // F*T tokens
  int ntt;               // ceil(F*T/64) token-order tiles
  // work items in segments of one head each (a head has at most two: special-row and patch-row
  // items), ordered longest item first; segment i covers blocks item_start[i] .. item_start[i+1]-1
  // and items item_base[i] ... of head order[i]
  int n_order;
  int16_t order[kMaxSegs];
  int item_start[kMaxSegs + 1];
  int item_base[kMaxSegs];
  int8_t pattern[kMaxHeads];
  int8_t slot[kMaxHeads];
};

__device__ inline float partner_max(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ inline float partner_sum(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// high word of a 32 x 32-bit product as one multiply instruction (the __umulhi library routine is
// an out-of-line call here, with the call's register saves, once per use)
__device__ __forceinline__ uint32_t mulhi_u32(uint32_t a, uint32_t b) { return (uint32_t)(((uint64_t)a * b) >> 32); }

struct Acc {
  f32x16 o[2][2];  // [dh][gq]: O^T rows 32*dh + (16*half + a), query 32*gq + col
  float m[2];      // reference maximum (raw score units) per query group
  float l[2];      // partial row sum over this lane's keys
  f32x4 ls;        // FAST walks: element gq = this lane's row sum of group gq from the matrix core
  s16x4 sel[2];    // 0/1 selector operands of those row sums (bf16 1.0 in the lanes of row gq)
};

// FAST row sums on the matrix core: v_mfma_f32_4x4x4_16b_bf16 computes, in each of its 16 blocks
// of four lanes, D[i][j] = sum_k A[i][k] B[k][j], with A row i held by lane 4b+i, B column j and D
// column j by lane 4b+j, and D row i in accumulator element i. With B = four P values of a lane
// and A = sel[gq] (ones in row gq only) the lane's own accumulator element gq gains the sum of its
// four values; two instructions take a P fragment (eight values). The P values are the bf16 ones
// that feed the PV product, as with the dot2 sums.
__device__ __forceinline__ void rowsum_mfma(Acc& A, const bf16x8& pf, int gq) {
  const u32x4 w = __builtin_bit_cast(u32x4, pf);
  const s16x4 lo = __builtin_bit_cast(s16x4, u32x2{w[0], w[1]});
  const s16x4 hi = __builtin_bit_cast(s16x4, u32x2{w[2], w[3]});
  A.ls = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A.sel[gq], lo, A.ls, 0, 0, 0);
  A.ls = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A.sel[gq], hi, A.ls, 0, 0, 0);
}

// end of a FAST pipelined walk: the matrix-core row sums join the lane's partial sums
__device__ __forceinline__ void fold_rowsums(Acc& A) {
  A.l[0] += A.ls[0];
  A.l[1] += A.ls[1];
  A.ls = f32x4{};
}

struct TileMask {
  bool need;     // some element of the tile is masked
  bool kspecial; // key tile lies in the special region
  int kt;        // key tile index
  int kvalid;    // patch tile: valid keys from key 0 of the tile
  int kframe;    // patch tile: frame of its keys
  int eff;       // pattern whose frame relation applies (DENSE / BLOCK_DYNAMIC: none)
};

// One staged key tile (NKH = 2: 64 keys, K rows 128 B, V rows 128 B) or half tile (NKH = 1:
// 32 keys, V rows 64 B); key0 is the first key of the staged keys within their 64-slot tile.
template <int NKH, typename Hook>
__device__ __forceinline__ void attend(const char* __restrict__ kst, const char* __restrict__ vst,
                                       const bf16x8 (&qfrag)[2][4], Acc& A, const int (&frow)[2],
                                       const TileMask& tm, const Geom& g, uint32_t nsmagic, int key0, int half,
                                       int col, float c, Hook&& hook) {
  f32x16 s[NKH][2];
  // S^T of the staged keys, masked; also re-run by the exact path below, which keeps s from
  // having to stay live next to P
  auto scores = [&]() {
#pragma unroll
    for (int kh = 0; kh < NKH; ++kh) s[kh][0] = s[kh][1] = f32x16{};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int chn = 4 * half + st;
#pragma unroll
      for (int kh = 0; kh < NKH; ++kh) {
        const int r = 32 * kh + col;
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kst + r * 128 + ((chn ^ swz8(r)) << 4));
        s[kh][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qfrag[0][st], s[kh][0], 0, 0, 0);
        s[kh][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qfrag[1][st], s[kh][1], 0, 0, 0);
      }
    }
    if (tm.need) {
#pragma unroll
      for (int kh = 0; kh < NKH; ++kh) {
#pragma unroll
        for (int a = 0; a < 16; ++a) {
          const int key = key0 + 32 * kh + 8 * (a >> 2) + 4 * half + (a & 3);
          bool ok;
          int fc;
          if (tm.kspecial) {
            // frame = slot / ns as a multiply-high with ceil(2^32 / ns), exact below 2^32 / ns
            // (magic 0: ns = 1)
            const uint32_t sl = (uint32_t)(tm.kt * 64 + key);
            ok = sl < (uint32_t)g.S;
            fc = nsmagic ? (int)mulhi_u32(sl, nsmagic) : (int)sl;
          } else {
            ok = key < tm.kvalid;
            fc = tm.kframe;
          }
#pragma unroll
          for (int gq = 0; gq < 2; ++gq) {
            bool okg = ok;
            if (tm.eff == SAF3R_FRAME_LOCAL) okg = okg && fc == frow[gq];
            else if (tm.eff == SAF3R_ANCHOR_LOCAL) okg = okg && (fc == 0 || fc == frow[gq]);
            else if (tm.eff == SAF3R_ANCHOR) okg = okg && fc == 0;
            if (!okg) s[kh][gq][a] = -__builtin_inff();
          }
        }
      }
    }
  };
  scores();
  // loads issued here wait in the memory pipeline while the score MFMAs execute
  __builtin_amdgcn_sched_barrier(0);
  hook();
  __builtin_amdgcn_sched_barrier(0);

  // P = exp2(s*c - m*c) against the row's reference maximum m, and this tile's partial row sums.
  // m is raised only when a tile's partial sum exceeds 2^64 (the first tile of a row with an
  // unmasked key, whose m is still -inf, always does): values up to 2^64 keep every bf16 P, every
  // fp32 sum and O finite, so no per-tile maximum is needed. The exact path then takes the tile's
  // row maximum, rescales O and l, and recomputes P.
  bf16x8 pf[2][2 * NKH];
  float ts[2];
  // row sums over the bf16-rounded P that the PV product uses, so l and O agree
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  auto exps = [&](int gq, float mc) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * NKH; ++j) {
      const int a0 = 8 * (j & 1);
#pragma unroll
      for (int u = 0; u < 8; u += 2) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j >> 1][gq][a0 + u], c, -mc));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j >> 1][gq][a0 + u + 1], c, -mc));
        const bf16x2 pr = {(__bf16)e0, (__bf16)e1};
        pf[gq][j][u] = pr[0];
        pf[gq][j][u + 1] = pr[1];
        t = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, t, false);
      }
    }
    ts[gq] = t;
  };
  // a row without a reference yet uses -2^127: unmasked keys then give +inf (and the exact
  // path), masked keys 0, and no inf - inf (NaN) ever forms
#pragma unroll
  for (int gq = 0; gq < 2; ++gq) exps(gq, A.m[gq] == -__builtin_inff() ? -0x1p127f : A.m[gq] * c);
  if (__ballot(ts[0] > 0x1p64f || ts[1] > 0x1p64f) != 0) {
    scores();
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      float mx = s[0][gq][0];
#pragma unroll
      for (int kh = 0; kh < NKH; ++kh)
#pragma unroll
        for (int a = 0; a < 16; ++a) mx = fmaxf(mx, s[kh][gq][a]);
      mx = partner_max(mx);
      const float m_new = fmaxf(A.m[gq], mx);
      const float alpha = A.m[gq] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f((A.m[gq] - m_new) * c);
      A.l[gq] *= alpha;
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        A.o[0][gq][a] *= alpha;
        A.o[1][gq][a] *= alpha;
      }
      A.m[gq] = m_new;
      exps(gq, m_new == -__builtin_inff() ? 0.f : m_new * c);
    }
  }
  A.l[0] += ts[0];
  A.l[1] += ts[1];

#pragma unroll
  for (int j = 0; j < 2 * NKH; ++j) {
    const int chn = 2 * j + half;
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) {
      const int r = 32 * dh + col;
      const bf16x8 vf = NKH == 2 ? *reinterpret_cast<const bf16x8*>(vst + r * 128 + ((chn ^ swz8(r)) << 4))
                                 : *reinterpret_cast<const bf16x8*>(vst + r * 64 + ((chn ^ swz4(r)) << 4));
      A.o[dh][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[0][j], A.o[dh][0], 0, 0, 0);
      A.o[dh][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[1][j], A.o[dh][1], 0, 0, 0);
    }
  }
}

// ---- single-range walks: software pipeline over 32-key half steps ------------------------------
// Half step h covers keys 32 * (h & 1) .. + 31 of the h / 2-th tile of the walk. One block of
// straight-line code runs the PV MFMAs of step h - 1, the score MFMAs of step h + 1 and the softmax
// of step h, one MFMA to one softmax group (2 fma, 2 exp, 1 convert), so a wave keeps the matrix
// unit busy while it computes exponentials instead of alternating between the two.

// K fragments of keys 32 kh .. 32 kh + 31 of a staged tile (128-byte rows, swz8)
__device__ __forceinline__ void load_k(const char* __restrict__ kst, int kh, bf16x8 (&kf)[4], int half, int col) {
  const int r = 32 * kh + col;
#pragma unroll
  for (int st = 0; st < 4; ++st)
    kf[st] = *reinterpret_cast<const bf16x8*>(kst + r * 128 + (((4 * half + st) ^ swz8(r)) << 4));
}
// V^T fragments of keys 32 kh .. 32 kh + 31 of a staged transposed tile (128-byte rows, swz8)
__device__ __forceinline__ void load_v(const char* __restrict__ vst, int kh, bf16x8 (&vf)[2][2], int half, int col) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) {
      const int r = 32 * dh + col, chn = 2 * (2 * kh + j) + half;
      vf[j][dh] = *reinterpret_cast<const bf16x8*>(vst + r * 128 + ((chn ^ swz8(r)) << 4));
    }
}

// Masks keys key0 + i >= kvalid of a half step (single-range walks: no frame relation applies).
__device__ __forceinline__ void mask_valid(f32x16 (&s)[2], int kvalid, int key0, int half) {
#pragma unroll
  for (int a = 0; a < 16; ++a) {
    const int key = key0 + 8 * (a >> 2) + 4 * half + (a & 3);
    if (key >= kvalid) s[0][a] = s[1][a] = -__builtin_inff();
  }
}

// a row without a reference maximum yet uses -2^127: unmasked keys then give +inf (and the exact
// path), masked keys 0, and no inf - inf (NaN) ever forms
__device__ __forceinline__ float ref_mc(float m, float c) { return m == -__builtin_inff() ? -0x1p127f : m * c; }

// P = exp2(s*c - mc) of one query group's 16 keys and their partial row sum over the bf16-rounded
// values the PV product uses (exact path)
__device__ __forceinline__ float exps_half(const f32x16& s, float c, float mc, bf16x8 (&p)[2]) {
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  float t = 0.f;
#pragma unroll
  for (int u = 0; u < 16; u += 2) {
    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u], c, -mc));
    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u + 1], c, -mc));
    const bf16x2 pr = {(__bf16)e0, (__bf16)e1};
    p[u >> 3][u & 7] = pr[0];
    p[u >> 3][(u & 7) + 1] = pr[1];
    t = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, t, false);
  }
  return t;
}

// The block of half step h: O += V(h-1) P(h-1), sn = K(h+1) Q^T, pn = P(h) from s with row sums ts.
// FAST: the head's Q rows carry the softmax scale and the walk keeps no reference maximum, so
// P = exp2(s) with no per-score arithmetic before the exponential (see walk_unsafe).
template <bool FAST>
__device__ __forceinline__ void half_block(const bf16x8 (&kf)[4], const bf16x8 (&vf)[2][2],
                                           const bf16x8 (&qfrag)[2][4], const f32x16 (&s)[2], f32x16 (&sn)[2],
                                           const bf16x8 (&p)[2][2], bf16x8 (&pn)[2][2], float (&ts)[2], Acc& A,
                                           float c) {
  const float mc0 = FAST ? 0.f : ref_mc(A.m[0], c), mc1 = FAST ? 0.f : ref_mc(A.m[1], c);
  sn[0] = sn[1] = f32x16{};
  auto matrix = [&](int i) {
    if (i < 8) {
      const int j = i >> 2, dh = (i >> 1) & 1, gq = i & 1;
      A.o[dh][gq] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[j][dh], p[gq][j], A.o[dh][gq], 0, 0, 0);
      if constexpr (FAST)
        if (dh == 1) rowsum_mfma(A, p[gq][j], gq);  // each P fragment once, after its second PV
    } else {
      const int k = i - 8, st = k >> 1, gq = k & 1;
      sn[gq] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qfrag[gq][st], sn[gq], 0, 0, 0);
    }
  };
  auto vector = [&](int i) {
    const int g2 = i >> 3, u = 2 * (i & 7);
    const float mc = g2 ? mc1 : mc0;
    const float e0 = __builtin_amdgcn_exp2f(FAST ? s[g2][u] : __builtin_fmaf(s[g2][u], c, -mc));
    const float e1 = __builtin_amdgcn_exp2f(FAST ? s[g2][u + 1] : __builtin_fmaf(s[g2][u + 1], c, -mc));
    const bf16x2 pr = {(__bf16)e0, (__bf16)e1};
    pn[g2][u >> 3][u & 7] = pr[0];
    pn[g2][u >> 3][(u & 7) + 1] = pr[1];
  };
  // fixed order: the first softmax group covers the LDS latency of the fragments, then each MFMA
  // is followed by one softmax group (scheduling barriers keep the compiler from regrouping)
  vector(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    matrix(i);
    if (i + 1 < 16) vector(i + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  // row sums of the rounded P (so l and O agree), as one burst of dot2 at the end: each dot2
  // waits for the matrix pipe, so spread between the MFMAs they would stall every one of them.
  // FAST walks summed P(h-1) on the matrix core above and never read ts.
  if constexpr (!FAST) {
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    ts[0] = ts[1] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int u = 0; u < 8; u += 2)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const bf16x2 pr = {pn[g][j][u], pn[g][j][u + 1]};
          ts[g] = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, ts[g], false);
        }
    asm volatile("" : "+v"(ts[0]), "+v"(ts[1]));
  } else {
    asm volatile("" : "+v"(A.ls));
  }
  // every result is due here: otherwise the compiler sinks the softmax (and MFMAs) past the
  // masking branch that follows, into blocks of their own, and nothing overlaps any more
  asm volatile("" : "+v"(pn[0][0]), "+v"(pn[0][1]), "+v"(pn[1][0]), "+v"(pn[1][1]));
  asm volatile("" : "+v"(sn[0]), "+v"(sn[1]));
  asm volatile("" : "+v"(A.o[0][0]), "+v"(A.o[0][1]), "+v"(A.o[1][0]), "+v"(A.o[1][1]));
}

// The reference maximum m moves only when a step's partial row sum exceeds 2^64 (the first step of
// a row with an unmasked key, whose m is still -inf, always does): values up to 2^64 keep every
// bf16 P, fp32 sum and O finite, so no per-step maximum is needed. The exact path takes the row
// maximum of s, rescales O (which then holds every step before h) and l, and recomputes P(h).
// The row sums a FAST walk (reference maximum fixed at 0) may end with: within [2^-64, 2^64] every
// P of the row is at most 2^64 and the row's largest P at least 2^-64 / n (no NaN passes).
// The test runs on the bits: for l >= 0 their order is the order of the values, and a NaN (which
// the matrix-core row sums give where a selector zero meets an infinite P, and which comparisons
// compiled without NaN semantics would not see) lies above 2^64 there, as does -0.
__device__ __forceinline__ bool in_fast_range(float l) {
  const uint32_t b = __builtin_bit_cast(uint32_t, l);
  return b >= 0x1F800000u && b <= 0x5F800000u;  // 2^-64, 2^64
}

// FAST walks (reference fixed at 0) check nothing per step: every P is non-negative, so a row sum
// that ends within [2^-64, 2^64] bounds every P of the row, and the end of the walk tests that.
template <bool FAST>
__device__ __forceinline__ void exact_fix(const f32x16 (&s)[2], bf16x8 (&pn)[2][2], float (&ts)[2], Acc& A,
                                          float c) {
  if constexpr (FAST) return;
  if (__ballot(ts[0] > 0x1p64f || ts[1] > 0x1p64f) == 0) return;
#pragma unroll
  for (int gq = 0; gq < 2; ++gq) {
    float mx = s[gq][0];
#pragma unroll
    for (int a = 1; a < 16; ++a) mx = fmaxf(mx, s[gq][a]);
    mx = partner_max(mx);
    const float m_new = fmaxf(A.m[gq], mx);
    const float alpha = A.m[gq] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f((A.m[gq] - m_new) * c);
    A.l[gq] *= alpha;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      A.o[0][gq][a] *= alpha;
      A.o[1][gq][a] *= alpha;
    }
    A.m[gq] = m_new;
    ts[gq] = exps_half(s[gq], c, m_new == -__builtin_inff() ? 0.f : m_new * c, pn[gq]);
  }
}

// Key-tile walk of a shared-mode group: up to four contiguous tile ranges (empty ones skipped),
// entered at any step and wrapping around. Patch tiles carry their block within the frame and
// their frame, advanced incrementally, so a step costs a few scalar instructions and no division.
// Every field is work-group uniform and lives in scalar registers.
struct Walk {
  int s0, l0, s1, l1, s2, l2, s3, l3;  // the ranges (length 0: empty)
  int count;
  int r, kt, rem;  // current range, current tile, tiles left in the range from kt on
  int b, f;        // patch tile: block within its frame, frame (b = -1 on special tiles)

  // ranges are selected by value, never through an indexed array: an array indexed at run time
  // would live in scratch memory, and values loaded from there count as per-lane values
  __device__ inline int rs(int i) const { return i == 0 ? s0 : i == 1 ? s1 : i == 2 ? s2 : s3; }
  __device__ inline int rl(int i) const { return i == 0 ? l0 : i == 1 ? l1 : i == 2 ? l2 : l3; }
  __device__ inline void init(int a0, int b0, int a1, int b1, int a2, int b2, int a3, int b3) {
    s0 = __builtin_amdgcn_readfirstlane(a0);
    l0 = __builtin_amdgcn_readfirstlane(max(b0, 0));
    s1 = __builtin_amdgcn_readfirstlane(a1);
    l1 = __builtin_amdgcn_readfirstlane(max(b1, 0));
    s2 = __builtin_amdgcn_readfirstlane(a2);
    l2 = __builtin_amdgcn_readfirstlane(max(b2, 0));
    s3 = __builtin_amdgcn_readfirstlane(a3);
    l3 = __builtin_amdgcn_readfirstlane(max(b3, 0));
    count = l0 + l1 + l2 + l3;
    r = kt = rem = b = f = 0;
  }
  __device__ inline void locate(const Geom& g) {
    if (kt >= g.nst) {
      f = (kt - g.nst) / g.NBf;
      b = kt - g.nst - f * g.NBf;
    } else {
      b = -1;
      f = 0;
    }
  }
  // position at step pos of the sequence (0 <= pos < count)
  __device__ inline void seek(int pos, const Geom& g) {
    r = 0;
    while (pos >= rl(r)) {  // ends: pos < count
      pos -= rl(r);
      ++r;
    }
    kt = rs(r) + pos;
    rem = rl(r) - pos;
    locate(g);
  }
  __device__ inline void next(const Geom& g) {
    if (--rem > 0) {
      ++kt;
      if (kt == g.nst) {
        b = 0;
        f = 0;
      } else if (b >= 0 && ++b == g.NBf) {
        b = 0;
        ++f;
      }
    } else {
      do r = (r + 1) & 3;
      while (rl(r) == 0);  // ends: count > 0
      kt = rs(r);
      rem = rl(r);
      locate(g);
    }
  }
  // mask description of the current tile for a shared-mode query tile
  __device__ inline TileMask mask(const Geom& g, int eff, bool frame_rel, bool qspecial) const {
    TileMask tm;
    tm.kt = kt;
    tm.eff = eff;
    tm.kspecial = kt < g.nst;
    if (tm.kspecial) {
      tm.kvalid = 64;
      tm.kframe = 0;
      tm.need = (kt + 1) * 64 > g.S || frame_rel;
    } else {
      tm.kframe = f;
      tm.kvalid = b == g.NBf - 1 ? g.P - 64 * b : 64;
      tm.need = tm.kvalid < 64 || (frame_rel && qspecial);
    }
    return tm;
  }
};

__device__ inline void store_rows(const AttnParams& p, const Acc& A, const int64_t (&qtok)[2], int h, int half) {
#pragma unroll
  for (int gq = 0; gq < 2; ++gq) {
    const float lt = partner_sum(A.l[gq]);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if (qtok[gq] >= 0) {
      uint32_t wv[16];
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        const bf16x2 x0 = {(__bf16)(A.o[0][gq][2 * a] * inv), (__bf16)(A.o[0][gq][2 * a + 1] * inv)};
        const bf16x2 x1 = {(__bf16)(A.o[1][gq][2 * a] * inv), (__bf16)(A.o[1][gq][2 * a + 1] * inv)};
        wv[a] = __builtin_bit_cast(uint32_t, x0);
        wv[8 + a] = __builtin_bit_cast(uint32_t, x1);
      }
      u32x4* o4 = reinterpret_cast<u32x4*>(p.out + qtok[gq] * p.out_stride + (int64_t)h * 64 + 16 * half);
      o4[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
      o4[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
      o4[4] = u32x4{wv[8], wv[9], wv[10], wv[11]};
      o4[5] = u32x4{wv[12], wv[13], wv[14], wv[15]};
    }
  }
}

// ---- walk pacing ------------------------------------------------------------------------------
// A walk starts at the position the wall clock divided by the step time points to. The step time of
// walk kind k (0: single-range walks, 1: split-mode waves) is the mean measured by the previous call:
// finishing walks add their elapsed ticks and steps to the caller's pace state (slot pace_acc), the
// next call reads them (slot pace_read) and clears the slot the call after it accumulates into.
// Reads and updates are vector atomics through L2; the state only steers walk starts, never results.
constexpr uint64_t kPaceMinSteps = 256;  // measured steps below this: use the default step time
constexpr int kPaceMinWalk = 16;         // walks shorter than this do not contribute
#ifndef SAF3R_PACE_SCALE_PCT
#define SAF3R_PACE_SCALE_PCT 100         // phase = measured mean step time * this / 100
#endif

__device__ inline uint64_t pace_phase(const AttnParams& p, int kind) {
  const uint64_t def = kind ? p.phase_split : p.phase_dense;
  if (!p.pace) return def;
  unsigned long long* s = p.pace + kind * 6 + p.pace_read * 2;
  const uint64_t ticks = __hip_atomic_load(s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t steps = __hip_atomic_load(s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (steps < kPaceMinSteps) return def;
  const uint64_t ph = ticks * SAF3R_PACE_SCALE_PCT / (steps * 100);
  return ph > 0 ? ph : 1;
}

__device__ inline void pace_add(const AttnParams& p, int kind, uint64_t t0, int steps) {
  if (!p.pace || steps < kPaceMinWalk) return;
  const uint64_t dt = __builtin_amdgcn_s_memrealtime() - t0;
  unsigned long long* s = p.pace + kind * 6 + p.pace_acc * 2;
  __hip_atomic_fetch_add(s, (unsigned long long)dt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_add(s + 1, (unsigned long long)steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A work item: head, pattern, item index within the head, first query tile, waves with a tile of
// their own, walk kind, and (BROADCAST) the frame whose rows it writes.
struct Item {
  int h, pat, it, qt0, nw, kind, bfr;
  bool tokord, framed;
};

__device__ inline Item decode_item(const AttnParams& p, int item) {
  const Geom& g = p.g;
  Item d;
  int oh = 0;
  while (oh + 1 < p.n_order && item >= p.item_start[oh + 1]) ++oh;
  d.h = p.order[oh];
  d.pat = p.pattern[d.h];
  d.it = item - p.item_start[oh] + p.item_base[oh];
  d.bfr = 0;
  const int pat = d.pat, it = d.it;
  const int ns4 = (g.nst + 3) >> 2;
  const int groups_pf = (g.NBf + 3) >> 2;
  d.tokord = pat == SAF3R_DENSE && ((p.tok_order >> d.h) & 1);
  d.framed = d.h < 64 && ((p.framed >> d.h) & 1);
  if (d.framed) {
    // four consecutive query tiles of one frame (the frame's last item may hold fewer)
    const int gpf = (g.NBT + 3) >> 2, f = it / gpf, gg = it - f * gpf;
    d.qt0 = f * g.NBT + 4 * gg;
    d.nw = min(4, g.NBT - 4 * gg);
    d.kind = kShared;
  } else if (pat == SAF3R_DENSE || pat == SAF3R_SKIP || pat == SAF3R_KEYSET) {
    d.qt0 = 4 * it;
    d.nw = min(4, (d.tokord ? p.ntt : g.NT) - d.qt0);
    d.kind = pat == SAF3R_SKIP ? kSkip : kShared;
  } else if (pat == SAF3R_BROADCAST) {
    // query tile qt of frame 0's compact rows, written for frame bfr
    const int nq = p.bcap / 64, gpf = (nq + 3) >> 2;
    d.bfr = it / gpf;
    d.qt0 = 4 * (it - d.bfr * gpf);
    d.nw = min(4, nq - d.qt0);
    d.kind = kShared;
  } else if (pat == SAF3R_TOKEN_DYNAMIC || pat == SAF3R_TOKEN_DYNAMIC_KEYSET || (pat == SAF3R_BLOCK_DYNAMIC && it < ns4)) {
    d.qt0 = 4 * it;
    d.nw = min(4, g.nst - d.qt0);
    d.kind = kShared;
  } else if (pat == SAF3R_BLOCK_DYNAMIC) {
    d.qt0 = g.nst + (it - ns4);
    d.nw = 4;  // four waves on one query tile
    d.kind = kSplit;
  } else if (it < g.nst) {
    d.qt0 = it;
    d.nw = 1;
    d.kind = kShared;
  } else {
    const int j = it - g.nst, f = j / groups_pf, gg = j % groups_pf;
    d.qt0 = g.nst + f * g.NBf + 4 * gg;
    d.nw = min(4, g.NBf - 4 * gg);
    d.kind = kShared;
  }
  return d;
}

// FAST marker of an item: feature 0 of row 0 of its first query tile (a row that always exists)
__device__ inline uint16_t* item_marker(const AttnParams& p, const Item& d) {
  const Geom& g = p.g;
  int64_t t0;
  if (d.pat == SAF3R_BROADCAST) t0 = (int64_t)d.bfr * g.T + d.qt0 * 64;
  else if (d.tokord) t0 = (int64_t)d.qt0 * 64;
  else if (d.framed) t0 = (int64_t)(d.qt0 / g.NBT) * g.T + (d.qt0 % g.NBT) * 64;
  else if (d.qt0 < g.nst) t0 = (int64_t)(d.qt0 * 64 / g.ns) * g.T + (d.qt0 * 64) % g.ns;
  else t0 = (int64_t)((d.qt0 - g.nst) / g.NBf) * g.T + g.ns + ((d.qt0 - g.nst) % g.NBf) * 64;
  return reinterpret_cast<uint16_t*>(p.out + t0 * p.out_stride + (int64_t)d.h * 64);
}

// The kernel body for work item `item` (uniform). FIXUP: walked again, exactly, because the main
// launch marked it.
template <bool FIXUP>
__device__ __forceinline__ void attn_body(const AttnParams& p, const int item) {
  __shared__ __align__(16) char ring[kRing];
  __shared__ int list[kMaxList];
  __shared__ int wcnt[4];
  __shared__ int uflag[4];
  __shared__ uint64_t t_start;

  const Geom& g = p.g;
  // the id builtins, not threadIdx / blockIdx: in a kernel this large the latter stay calls, whose
  // results the compiler must treat as per-lane values, and everything derived from the work-group
  // id (the whole work-item decode and key walk) would run on the vector unit
  const int tid = __builtin_amdgcn_workitem_id_x();
  const int lane = tid & 63, half = lane >> 5, col = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform
  if (!FIXUP && item == 0 && tid < 4 && p.pace) {  // the slot the next call accumulates into starts at zero
    unsigned long long* z = p.pace + (tid >> 1) * 6 + p.pace_zero * 2 + (tid & 1);
    __hip_atomic_store(z, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- decode the work item (uniform) ----
  const Item d = decode_item(p, item);
  const int h = d.h, pat = d.pat, qt0 = d.qt0, nw = d.nw, kind = d.kind;
  const int bfr = d.bfr;  // BROADCAST: the frame whose rows the item writes
  const bool tokord = d.tokord, framed = d.framed;
  const bool wactive = w < nw;
  const int qt = kind == kSplit ? qt0 : qt0 + (wactive ? w : 0);
  const bool qspecial = pat != SAF3R_BROADCAST && !tokord && !framed && qt < g.nst;
  // query frame and the tile's position within it (framed: every wave's tile is in qt0's frame)
  const int qf = framed ? qt0 / g.NBT : qspecial ? 0 : (qt - g.nst) / g.NBf;
  const int qb = framed ? qt - qf * g.NBT : qspecial ? 0 : (qt - g.nst) % g.NBf;
  const bool writer = kind == kSplit ? true : wactive;

  // output token (or -1) and frame of the lane's two query rows; evaluated where they are used
  // rather than held in registers through the key walk
  auto row_info = [&](int64_t(&qtok)[2], int(&frow)[2]) {
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      const int r = 32 * gq + col;
      if (pat == SAF3R_BROADCAST) {
        const int i = qt * 64 + r;
        qtok[gq] = (writer && i < g.T) ? (int64_t)bfr * g.T + i : -1;
        frow[gq] = bfr;
      } else if (tokord) {
        const int i = qt * 64 + r;
        qtok[gq] = (writer && i < p.ntok) ? (int64_t)i : -1;
        frow[gq] = 0;
      } else if (framed) {
        const int i = qb * 64 + r;
        qtok[gq] = (writer && i < g.T) ? (int64_t)qf * g.T + i : -1;
        frow[gq] = qf;
      } else if (qspecial) {
        const int64_t sl = (int64_t)qt * 64 + r;
        qtok[gq] = (writer && sl < g.S) ? (sl / g.ns) * g.T + sl % g.ns : -1;
        frow[gq] = g.ns > 0 ? (int)(sl / g.ns) : 0;
      } else {
        const int pp = qb * 64 + r;
        qtok[gq] = (writer && pp < g.P) ? (int64_t)qf * g.T + g.ns + pp : -1;
        frow[gq] = qf;
      }
    }
  };
  auto store = [&](const Acc& A) {
    int64_t qtok[2];
    int frow[2];
    row_info(qtok, frow);
    store_rows(p, A, qtok, h, half);
  };
  const int64_t head_base = (int64_t)h * g.L;

  if (kind == kSkip) {
    int64_t qtok[2];
    int frow[2];
    row_info(qtok, frow);
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      if (qtok[gq] >= 0) {
        u32x4* o4 = reinterpret_cast<u32x4*>(p.out + qtok[gq] * p.out_stride + (int64_t)h * 64 + 16 * half);
        const u32x4 z = {0, 0, 0, 0};
        o4[0] = z;
        o4[1] = z;
        o4[4] = z;
        o4[5] = z;
      }
    }
    return;
  }

  // Heads whose Q rows carry the softmax scale (q * scale * log2 e, rounded once when packed) walk
  // in those units (c = 1) and without a reference maximum (FAST: P = exp2(s)) when every stored
  // row's sum ends within [2^-64, 2^64] (scores within about 64 units of 0). A FAST item whose rows
  // do not stores nothing but a marker, 0xFFFF (a NaN, which finite inputs never give) in
  // feature 0 of its first row, and the launch that follows (FIXUP) walks the marked items again
  // with the exact reference maximum.
  const bool qpre = h < 64 && ((p.q_pre >> h) & 1);
  const bool fast = qpre && !FIXUP;
  const float c = qpre ? 1.f : p.c;
  // (the marker address is recomputed where it is used rather than held through the walk)
  auto marker = [&]() { return item_marker(p, d); };
  // ---- Q fragments: lane holds features 32*half .. 32*half+31 of rows 32*gq + col ----
  bf16x8 qfrag[2][4];
  const __bf16* qrows = pat == SAF3R_BROADCAST ? p.bq + (int64_t)p.slot[h] * p.bcap * 64 : p.q + head_base * 64;
  // the tile index through an empty asm: the row numbers computed here must not be kept for the
  // output rows after the walk (a 64-bit value held through the key loops was spilled in them)
  int qtq = qt;
  asm volatile("" : "+s"(qtq));
#pragma unroll
  for (int gq = 0; gq < 2; ++gq) {
    const u32x4* qsrc = reinterpret_cast<const u32x4*>(qrows + ((int64_t)qtq * 64 + 32 * gq + col) * 64 + 32 * half);
#pragma unroll
    for (int s = 0; s < 4; ++s) qfrag[gq][s] = __builtin_bit_cast(bf16x8, qsrc[s]);
  }

  Acc A;
  auto init_acc = [&](bool fast) {
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      A.o[a][0] = A.o[a][1] = f32x16{};
      A.m[a] = fast ? 0.f : -__builtin_inff();
      A.l[a] = 0.f;
      const short one = (lane & 3) == a ? (short)0x3F80 : (short)0;  // bf16 1.0 in row a's lanes
      A.sel[a] = s16x4{one, one, one, one};
    }
    A.ls = f32x4{};
  };
  // FAST end of a walk: true (work-group uniform) when the item must be walked again exactly
  auto walk_unsafe = [&]() -> bool {
    int64_t qtok[2];
    int frow[2];
    row_info(qtok, frow);
    bool low = false;
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) low |= qtok[gq] >= 0 && !in_fast_range(partner_sum(A.l[gq]));
    const bool bad = __ballot(low) != 0;
    if (lane == 0) uflag[w] = bad ? 1 : 0;
    __syncthreads();
    return (uflag[0] | uflag[1] | uflag[2] | uflag[3]) != 0;
  };

  if (kind == kShared) {
    // The shared-mode walk, instantiated separately for KEYSET heads (compact key-set tiles) and
    // for every other pattern, so neither carries the other's state in registers.
    auto shared_walk = [&](auto ks_tag, auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
    init_acc(FAST);
    // stores the rows, or (FAST, out of range) marks the item for the exact walk
    auto finish = [&]() {
      if constexpr (FAST) {
        if (walk_unsafe()) {
          if (tid == 0) *marker() = 0xFFFFu;
          return;
        }
      }
      store(A);
    };
    // ---- key-tile sequence (uniform) ----
    Walk wk;
    bool frame_rel = false, rel_patch = false;
    int seg_s = 0, seg_l = 0;  // own-frame patch tiles of a frame-relative patch-row item
    constexpr bool keyset = decltype(ks_tag)::value;
    const int eff = (pat == SAF3R_DENSE || pat == SAF3R_TOKEN_DYNAMIC || pat == SAF3R_BLOCK_DYNAMIC || keyset)
                        ? SAF3R_DENSE
                        : pat;
    // KEYSET heads walk the compact tiles of their key set, key k of the set being slot k there;
    // BROADCAST heads walk frame 0's compact K with the V tiles of the item's frame; token-order
    // DENSE heads walk their own rows, every token a key
    int ks_keys = 0;
    if constexpr (keyset)
      ks_keys = __builtin_amdgcn_readfirstlane(pat == SAF3R_BROADCAST ? g.T
                                               : tokord               ? p.ntok
                                                                      : min(p.ks_count[p.slot[h]], (int)p.ks_cap));
    // framed heads: frame 0's tiles (ANCHOR, and first for ANCHOR_LOCAL), then the query frame's
    // (FRAME_LOCAL, and ANCHOR_LOCAL from frame 1 on), each frame NBT tiles with only its last partial
    const bool two = framed && pat == SAF3R_ANCHOR_LOCAL && qf != 0;
    if constexpr (keyset) {
      wk.init(0, (ks_keys + 63) / 64, 0, 0, 0, 0, 0, 0);
    } else if (eff == SAF3R_DENSE) {
      wk.init(0, g.NT, 0, 0, 0, 0, 0, 0);
    } else if (framed) {
      wk.init(pat == SAF3R_FRAME_LOCAL ? qf * g.NBT : 0, g.NBT, two ? qf * g.NBT : 0, two ? g.NBT : 0, 0, 0, 0, 0);
    } else {
      frame_rel = true;
      int f0, f1;
      if (qt0 < g.nst) {
        const int last = min(g.S, (qt0 + nw) * 64) - 1;
        f0 = (qt0 * 64) / g.ns;
        f1 = last / g.ns;
      } else {
        f0 = f1 = (qt0 - g.nst) / g.NBf;
      }
      const bool need_anchor = (pat == SAF3R_ANCHOR_LOCAL || pat == SAF3R_ANCHOR);
      const bool need_local = (pat != SAF3R_ANCHOR);
      const bool has_sp = g.ns > 0;
      const int ls0 = has_sp ? (f0 * g.ns) / 64 : 0;
      const int ls1 = has_sp ? ((f1 + 1) * g.ns - 1) / 64 : -1;
      const bool anc_sp = has_sp && need_anchor && !(need_local && ls0 == 0);
      const bool anc_pt = need_anchor && !(need_local && f0 == 0);
      // ranges: frame 0's special tiles, the item's frames' special tiles, frame 0's patch tiles,
      // the item's frames' patch tiles. A patch-row item (one frame) walks its own frame's patch
      // tiles (only the last one partial) in the pipelined single-range walk and the other ranges
      // here, with per-key frame masks.
      rel_patch = qt0 >= g.nst && need_local;
      wk.init(0, anc_sp ? (g.ns - 1) / 64 + 1 : 0,
              ls0, (has_sp && need_local) ? ls1 - ls0 + 1 : 0,
              g.nst, anc_pt ? g.NBf : 0,
              g.nst + f0 * g.NBf, need_local && !rel_patch ? (f1 - f0 + 1) * g.NBf : 0);
      if (rel_patch) {
        seg_s = __builtin_amdgcn_readfirstlane(g.nst + f0 * g.NBf);
        seg_l = __builtin_amdgcn_readfirstlane(g.NBf);
      }
    }
    const int count = wk.count;
    int rot = 0;
    const bool paced = eff == SAF3R_DENSE && p.phase_dense > 0 && count > 0;
    if (paced) {
      // one clock reading per work-group: the four waves share the ring and must agree; the start
      // time waits in LDS for the pace update at the end (no registers held through the walk)
      if (tid == 0) {
        const uint64_t t = __builtin_amdgcn_s_memrealtime();
        t_start = t;
        wcnt[0] = (int)((t / pace_phase(p, 0)) % (uint64_t)count);
      }
      __syncthreads();
      rot = __builtin_amdgcn_readfirstlane(wcnt[0]);  // an LDS value, uniform: keep the walk scalar
    }
    if (count > 0) wk.seek(rot, g);
    Walk wi = wk;  // the tiles to load run two steps ahead of the tiles consumed

    // thread tid owns 16-byte chunks tid and tid + 256 of the K and the V tile (64 rows of 128 B,
    // same offsets for both); LDS chunk position P holds row P/8, global chunk (P % 8) ^ swz8(row)
    // (unsigned 32-bit offsets from a uniform base: the loads take the scalar-base address form)
    // (chunk tid + 256 is row tid/8 + 32 with the same swizzle: offset + 4096)
    uint32_t dofs;
    {
      const int r = tid >> 3;
      dofs = (uint32_t)(r * 128 + (((tid & 7) ^ swz8(r)) << 4));
    }
    const char* kbase = reinterpret_cast<const char*>(p.k + head_base * 64);
    const char* vbase = reinterpret_cast<const char*>(p.v + head_base * 64);
    if constexpr (keyset) {
      if (pat == SAF3R_BROADCAST) {
        kbase = reinterpret_cast<const char*>(p.bk + (int64_t)p.slot[h] * p.bcap * 64);
        vbase = reinterpret_cast<const char*>(p.bv + ((int64_t)p.slot[h] * g.F + bfr) * p.bcap * 64);
      } else if (tokord) {
        // token-order DENSE head: its own packed rows, walked like a key set of all F*T tokens
      } else {
        kbase = reinterpret_cast<const char*>(p.kc + (int64_t)p.slot[h] * p.ks_cap * 64);
        vbase = reinterpret_cast<const char*>(p.vc + (int64_t)p.slot[h] * p.ks_cap * 64);
      }
    }
    auto issue = [&](int stage) {
      const char* kb = kbase + (int64_t)wi.kt * 8192;
      const char* vb = vbase + (int64_t)wi.kt * 8192;
      char* st = ring + stage * 16384 + 64 * w * 16;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint32_t o = dofs;
        const char* bk = kb + 4096 * u;
        const char* bv = vb + 4096 * u;
        asm volatile("" : "+v"(o), "+s"(bk), "+s"(bv));  // scalar-base address form (see split mode)
        __builtin_amdgcn_global_load_lds((const void*)(bk + o), (lds_void*)(st + 4096 * u), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(bv + o), (lds_void*)(st + 8192 + 4096 * u), 16, 0, 0);
      }
      wi.next(g);
    };

    if (keyset || eff == SAF3R_DENSE || rel_patch || framed) {
      // ---- single-range walk: tiles rot, rot + 1, ... (mod count), only partial tiles masked ----
      // (dense and key-set walks: tiles 0 .. count-1 entered at rot; patch-row items of
      // frame-relative heads: their own frame's patch tiles, then the frame-relative walk below)
      // Control is kept to a few scalar selects per tile: the loop runs four tiles per trip so
      // that every stage offset is a constant, waves without a query tile of their own compute
      // on a duplicate (their rows are not stored), and the tile position and its valid-key
      // count advance without branches.
      // (framed heads: no special tiles, NBT tiles per frame, T - 64 (NBT - 1) valid keys in the last)
      const int nst = framed ? 0 : g.nst, NBf = framed ? g.NBT : g.NBf;
      const int lastv = framed ? g.T - 64 * (NBf - 1) : g.P - 64 * (NBf - 1);  // valid keys, last tile of a frame
      const int sbeg = rel_patch ? seg_s : framed ? wk.s0 : 0;
      const int cnt = rel_patch ? seg_l : count;
      // the tile after which the walk continues at jto: the end of the range (wrapping to its start),
      // or for a framed two-frame walk the end of frame 0 (continuing at the query frame)
      const int jfrom = two ? g.NBT : sbeg + cnt, jto = two ? wk.s1 : sbeg;
      int kt = (rel_patch || framed) ? sbeg : rot, bk = -1;  // consumed tile and its block within its frame
      if constexpr (!keyset) bk = kt >= nst ? (kt - nst) % NBf : -1;
      auto kvalid_of = [&]() -> int {
        if constexpr (keyset) return min(64, ks_keys - 64 * kt);
        else return kt < nst ? min(64, g.S - 64 * kt) : (bk == NBf - 1 ? lastv : 64);
      };
      auto advance = [&]() {
        kt = kt + 1 == jfrom ? jto : kt + 1;
        if constexpr (!keyset) bk = kt < nst ? -1 : (kt == nst || bk + 1 == NBf ? 0 : bk + 1);
      };
      int kti = kt;  // next tile to load
      auto issue_at = [&](int stage) {
        const char* kb = kbase + (int64_t)kti * 8192;
        const char* vb = vbase + (int64_t)kti * 8192;
        char* st = ring + stage * 16384 + 64 * w * 16;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          uint32_t o = dofs;
          const char* bk = kb + 4096 * u;
          const char* bv = vb + 4096 * u;
          asm volatile("" : "+v"(o), "+s"(bk), "+s"(bv));  // scalar-base address form (see split mode)
          __builtin_amdgcn_global_load_lds((const void*)(bk + o), (lds_void*)(st + 4096 * u), 16, 0, 0);
          __builtin_amdgcn_global_load_lds((const void*)(bv + o), (lds_void*)(st + 8192 + 4096 * u), 16, 0, 0);
        }
        kti = kti + 1 == jfrom ? jto : kti + 1;
      };
      if (cnt == 0) {
        store(A);
        return;
      }
      wait_vm<0>();  // Q fragments landed; from here vmcnt counts ring loads only
      for (int u = 0; u < 3; ++u)
        if (u < cnt) issue_at(u);
      if (cnt >= 3) wait_vm<8>();
      else if (cnt == 2) wait_vm<4>();
      else wait_vm<0>();
      barrier_only();
      f32x16 s_cur[2], s_nxt[2];
      bf16x8 pc[2][2], pn[2][2], kf[4], vf[2][2];
      float ts[2];
      int kv_cur = kvalid_of();
      load_k(ring, 0, kf, half, col);
      s_cur[0] = s_cur[1] = f32x16{};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        s_cur[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qfrag[0][st], s_cur[0], 0, 0, 0);
        s_cur[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qfrag[1][st], s_cur[1], 0, 0, 0);
      }
      if (kv_cur < 64) mask_valid(s_cur, kv_cur, 0, half);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          pc[j][x] = bf16x8{};
          vf[j][x] = bf16x8{};
        }
      for (int t0 = 0; t0 < cnt; t0 += 4) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = t0 + v;
          if (t >= cnt) break;
          // half step 2t: PV of tile t-1 keys 32..63, scores of tile t keys 32..63
          if (v > 0 || t0 > 0) load_v(ring + ((v + 3) & 3) * 16384 + 8192, 1, vf, half, col);
          load_k(ring + v * 16384, 1, kf, half, col);
          half_block<FAST>(kf, vf, qfrag, s_cur, s_nxt, pc, pn, ts, A, c);
          if (kv_cur < 64) mask_valid(s_nxt, kv_cur, 32, half);
          exact_fix<FAST>(s_cur, pn, ts, A, c);
          if constexpr (!FAST) {
            A.l[0] += ts[0];
            A.l[1] += ts[1];
          }
          advance();
          const int kv_nxt = kvalid_of();  // tile t + 1 (past the end: never read)
          if (t + 2 < cnt) wait_vm<4>();
          else wait_vm<0>();
          barrier_only();
          if (t + 3 < cnt) issue_at((v + 3) & 3);
          // half step 2t+1: PV of tile t keys 0..31, scores of tile t + 1 keys 0..31
          load_v(ring + v * 16384 + 8192, 0, vf, half, col);
          load_k(ring + ((v + 1) & 3) * 16384, 0, kf, half, col);
          half_block<FAST>(kf, vf, qfrag, s_nxt, s_cur, pn, pc, ts, A, c);
          if (kv_nxt < 64) mask_valid(s_cur, kv_nxt, 0, half);
          exact_fix<FAST>(s_nxt, pc, ts, A, c);
          if constexpr (!FAST) {
            A.l[0] += ts[0];
            A.l[1] += ts[1];
          }
          kv_cur = kv_nxt;
        }
      }
      load_v(ring + ((cnt - 1) & 3) * 16384 + 8192, 1, vf, half, col);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int dh = 0; dh < 2; ++dh) {
          A.o[dh][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[j][dh], pc[0][j], A.o[dh][0], 0, 0, 0);
          A.o[dh][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[j][dh], pc[1][j], A.o[dh][1], 0, 0, 0);
        }
      if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          rowsum_mfma(A, pc[0][j], 0);
          rowsum_mfma(A, pc[1][j], 1);
        }
        fold_rowsums(A);
      }
      if (!rel_patch) {
        if (tid == 0 && paced) pace_add(p, 0, t_start, cnt);
        finish();
        return;
      }
      __syncthreads();  // every wave is done with the ring before the frame-relative walk reuses it
    }

    // ---- frame-relative walks (up to four ranges, frame masks): one tile per attend step ----
    int64_t qtok_unused[2];
    int frow[2];
    row_info(qtok_unused, frow);
    wait_vm<0>();  // Q fragments landed; from here vmcnt counts ring loads only
    // tiles move in pairs: pair i+1 loads into the two free stages while pair i is consumed,
    // one barrier per pair
    if (count > 0) issue(0);
    if (count > 1) issue(1);
    for (int n = 0; n < count; n += 2) {
      wait_vm<0>();
      barrier_only();
      if (!wactive) {
        if (n + 2 < count) issue((n + 2) % kStages);
        if (n + 3 < count) issue((n + 3) % kStages);
        continue;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (n + u < count) {
          const TileMask tm = wk.mask(g, eff, frame_rel, qspecial);
          const char* kst = ring + ((n + u) % kStages) * 16384;
          attend<2>(kst, kst + 8192, qfrag, A, frow, tm, g, p.nsmagic, 0, half, col, c, [&]() {
            if (n + 2 + u < count) issue((n + 2 + u) % kStages);
          });
          wk.next(g);
        }
      }
    }
    finish();
    };
    auto run = [&](auto ks_tag) {
      if (fast) shared_walk(ks_tag, std::true_type{});
      else shared_walk(ks_tag, std::false_type{});
    };
    if (pat == SAF3R_KEYSET || pat == SAF3R_TOKEN_DYNAMIC_KEYSET || pat == SAF3R_BROADCAST || tokord)
      run(std::true_type{});
    else run(std::false_type{});
    return;
  }

  // ================= split mode: one query tile, block list split across the four waves ======
  {
    // compact the selection row into LDS (drop invalid entries, keep order); an entry holds the
    // key tile and the number of valid keys of its block: tile << 7 | valid (1..64)
    const int32_t* srow = p.sel + ((int64_t)p.slot[h] * ((int64_t)g.F * g.NBf) + (qt - g.nst)) * p.sel_width;
    int total = 0;
    for (int c0 = 0; c0 < p.sel_width; c0 += 256) {
      const int j = c0 + tid;
      const int v = j < p.sel_width ? srow[j] : -1;
      const bool ok = v >= 0 && v < g.F * g.NBf;
      const uint64_t m = __ballot(ok);
      const int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
      if (lane == 0) wcnt[w] = __popcll(m);
      __syncthreads();
      int off = total;
      for (int i = 0; i < w; ++i) off += wcnt[i];
      if (ok && off + pre < kMaxList) list[off + pre] = ((g.nst + v) << 7) | min(64, g.P - 64 * (v % g.NBf));
      total += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
      __syncthreads();
    }
    total = min(total, kMaxList);
    // wave w takes list positions w, w + 4, w + 8, ...: with lists in frame-major order, the four
    // waves (and, through the clock phase, every resident work-group) advance through the key
    // frames together
    const int nw = total > w ? (total - w + 3) >> 2 : 0;
    int i0 = 0;
    uint64_t t_split = 0;
    if (p.phase_split > 0 && nw > 0) {
      t_split = __builtin_amdgcn_s_memrealtime();
      i0 = (int)((t_split / pace_phase(p, 1)) % (uint64_t)nw);
    }
    i0 = __builtin_amdgcn_readfirstlane(i0);
    auto entry = [&](int i) {
      int ii = i + i0;
      if (ii >= nw) ii -= nw;
      return __builtin_amdgcn_readfirstlane(list[w + 4 * ii]);
    };

    // Half-step stream of this wave: every listed block takes two 32-key half steps (a block with
    // at most 32 valid keys has an all-masked second half), software-pipelined as in the
    // single-range walk. The wave's 16 KB are two slots, one per half: slot hh holds K and V^T of
    // half hh of a block, 4 KB each. At the end of half step h the wave loads K of step h + 3 and
    // V of step h + 1 into the regions step h has just finished with; past the end of the list
    // the last block is loaded again, so every step issues the same 8 loads a lane and one
    // vmcnt wait serves every step. Per-lane byte offsets of the 16-byte chunks a lane moves:
    // K half = 32 rows x 8 chunks, V half = 64 rows x 4 chunks of 128-byte rows.
    // Lane offsets of the 16-byte chunks: K chunk u of a lane = row 8u + lane/8, whose swizzle
    // differs between even and odd u only (2 offsets + multiples of 1024); V chunk u = row
    // 16u + lane/4, whose swizzle does not depend on u (1 offset + multiples of 2048). The
    // instruction's immediate offset moves the global and the LDS address alike, so K chunks u and
    // u + 2 share one base, one lane offset and one M0 (immediate 2048), and V chunks 2i and 2i + 1
    // share a base and M0 with lane offsets vo and vo + 1024 (immediate 1024: global +2048, LDS
    // +1024). The offsets pass through an empty asm so that the compiler cannot fold them into
    // hoisted 64-bit per-lane addresses (two registers per load held through the loop): the loads
    // keep the scalar-base form, uniform address plus 32-bit lane offset.
    uint32_t ko[2], vo;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int P = 64 * u + lane, r = P >> 3;
      ko[u] = (uint32_t)(r * 128 + (((P & 7) ^ swz8(r)) << 4));
    }
    {
      const int i = lane >> 2;
      vo = (uint32_t)(i * 128 + (((lane & 3) ^ swz4(i)) << 4));
    }
    const uint32_t vo1 = vo + 1024;
    const char* kbase = reinterpret_cast<const char*>(p.k + head_base * 64);
    const char* vbase = reinterpret_cast<const char*>(p.v + head_base * 64);
    char* slots = ring + w * 16384;
    auto issue_k = [&](int e, int hh) {
      const char* kb = kbase + (int64_t)(e >> 7) * 8192 + hh * 4096;
      char* st = slots + hh * 8192;
      asm volatile("" : "+s"(kb));
      uint32_t o0 = ko[0], o1 = ko[1], o2 = ko[0], o3 = ko[1];
      asm volatile("" : "+v"(o0), "+v"(o1), "+v"(o2), "+v"(o3));
      __builtin_amdgcn_global_load_lds((const void*)(kb + o0), (lds_void*)st, 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(kb + o1), (lds_void*)(st + 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(kb + o2), (lds_void*)st, 16, 2048, 0);
      __builtin_amdgcn_global_load_lds((const void*)(kb + o3), (lds_void*)(st + 1024), 16, 2048, 0);
    };
    auto issue_v = [&](int e, int hh) {
      const char* vb = vbase + (int64_t)(e >> 7) * 8192 + hh * 64;
      char* st = slots + hh * 8192 + 4096;
      const char* b0 = vb;
      const char* b1 = vb + 4096;
      uint32_t o0 = vo, o1 = vo1, o2 = vo, o3 = vo1;
      asm volatile("" : "+v"(o0), "+v"(o1), "+v"(o2), "+v"(o3), "+s"(b0), "+s"(b1));
      __builtin_amdgcn_global_load_lds((const void*)(b0 + o0), (lds_void*)st, 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(b0 + o1), (lds_void*)st, 16, 1024, 0);
      __builtin_amdgcn_global_load_lds((const void*)(b1 + o2), (lds_void*)(st + 2048), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(b1 + o3), (lds_void*)(st + 2048), 16, 1024, 0);
    };
    // V^T fragments of a staged half (64-byte rows, swz4)
    auto load_vh = [&](const char* vst, bf16x8(&vf)[2][2]) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int dh = 0; dh < 2; ++dh) {
          const int r = 32 * dh + col, chn = 2 * j + half;
          vf[j][dh] = *reinterpret_cast<const bf16x8*>(vst + r * 64 + ((chn ^ swz4(r)) << 4));
        }
    };

    // the wave's walk over its list positions; FAST: true when the wave must walk them again exactly
    // (each wave's partial result is merged with its own reference maximum below)
    auto split_walk = [&](auto fast_tag) -> bool {
    constexpr bool FAST = decltype(fast_tag)::value;
    init_acc(FAST);
    wait_vm<0>();
    if (nw > 0) {
      const auto ent = [&](int i) { return entry(min(i, nw - 1)); };
      int e0 = ent(0), e1 = ent(1), e2 = ent(2);
      issue_k(e0, 0);
      issue_k(e0, 1);
      issue_v(e0, 0);
      wait_vm<8>();
      f32x16 s_cur[2], s_nxt[2];
      bf16x8 pc[2][2], pn[2][2], kf[4], vf[2][2];
      float ts[2];
      load_k(slots, 0, kf, half, col);
      s_cur[0] = s_cur[1] = f32x16{};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        s_cur[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qfrag[0][st], s_cur[0], 0, 0, 0);
        s_cur[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qfrag[1][st], s_cur[1], 0, 0, 0);
      }
      if ((e0 & 127) < 32) mask_valid(s_cur, e0 & 127, 0, half);
      issue_k(e1, 0);  // the K fragments above have been read: slot 0's K is free
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          pc[j][x] = bf16x8{};
          vf[j][x] = bf16x8{};
        }
      for (int t = 0; t < nw; ++t) {
        // half step 2t: PV of block t-1 half 1, scores of block t half 1, softmax of block t half 0
        wait_vm<8>();
        if (t > 0) load_vh(slots + 8192 + 4096, vf);
        load_k(slots + 8192, 0, kf, half, col);
        half_block<FAST>(kf, vf, qfrag, s_cur, s_nxt, pc, pn, ts, A, c);
        issue_k(e1, 1);
        issue_v(e0, 1);
        const int kv0 = e0 & 127;
        if (kv0 < 64) mask_valid(s_nxt, kv0, 32, half);
        exact_fix<FAST>(s_cur, pn, ts, A, c);
        if constexpr (!FAST) {
          A.l[0] += ts[0];
          A.l[1] += ts[1];
        }
        // half step 2t+1: PV of block t half 0, scores of block t+1 half 0, softmax of block t half 1
        wait_vm<8>();
        load_vh(slots + 4096, vf);
        load_k(slots, 0, kf, half, col);
        half_block<FAST>(kf, vf, qfrag, s_nxt, s_cur, pn, pc, ts, A, c);
        issue_k(e2, 0);
        issue_v(e1, 0);
        const int kv1 = e1 & 127;
        if (kv1 < 32) mask_valid(s_cur, kv1, 0, half);
        exact_fix<FAST>(s_nxt, pc, ts, A, c);
        if constexpr (!FAST) {
          A.l[0] += ts[0];
          A.l[1] += ts[1];
        }
        e0 = e1;
        e1 = e2;
        e2 = ent(t + 3);
      }
      if (lane == 0 && t_split) pace_add(p, 1, t_split, nw);
      // PV of the last block's second half
      wait_vm<0>();
      load_vh(slots + 8192 + 4096, vf);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int dh = 0; dh < 2; ++dh) {
          A.o[dh][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[j][dh], pc[0][j], A.o[dh][0], 0, 0, 0);
          A.o[dh][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[j][dh], pc[1][j], A.o[dh][1], 0, 0, 0);
        }
      if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          rowsum_mfma(A, pc[0][j], 0);
          rowsum_mfma(A, pc[1][j], 1);
        }
        fold_rowsums(A);
        bool low = false;
#pragma unroll
        for (int gq = 0; gq < 2; ++gq) low |= !in_fast_range(partner_sum(A.l[gq]));
        return __ballot(low) != 0;
      }
    }
    return false;
    };
    const bool unsafe = fast ? split_walk(std::true_type{}) : split_walk(std::false_type{});

    // ---- merge the four partial results through LDS ----
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) A.l[gq] = partner_sum(A.l[gq]);
    if (lane == 0) uflag[w] = unsafe ? 1 : 0;
    __syncthreads();  // every wave is done with its slots and with the list
    if (uflag[0] | uflag[1] | uflag[2] | uflag[3]) {  // a FAST wave left the range: the tile is walked again
      if (tid == 0) *marker() = 0xFFFFu;
      return;
    }
    float* obuf = reinterpret_cast<float*>(ring) + w * 4096;  // [64 rows][64 d] fp32 per wave
    float* mls = reinterpret_cast<float*>(list);                // m[4][64], l[4][64]
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      const int row = 32 * gq + col;
#pragma unroll
      for (int dh = 0; dh < 2; ++dh) {
        f32x4* dst = reinterpret_cast<f32x4*>(obuf + row * 64 + 32 * dh + 16 * half);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          dst[q4] = f32x4{A.o[dh][gq][4 * q4], A.o[dh][gq][4 * q4 + 1], A.o[dh][gq][4 * q4 + 2], A.o[dh][gq][4 * q4 + 3]};
      }
      if (half == 0) {
        mls[w * 64 + row] = A.m[gq];
        mls[256 + w * 64 + row] = A.l[gq];
      }
    }
    __syncthreads();
    const int row = tid >> 2, d0 = (tid & 3) * 16;
    int64_t tok;
    if (qspecial) tok = -1;  // split mode only serves patch tiles
    else {
      const int pp = qb * 64 + row;
      tok = pp < g.P ? (int64_t)qf * g.T + g.ns + pp : -1;
    }
    float mw[4], M = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mw[i] = mls[i * 64 + row];
      M = fmaxf(M, mw[i]);
    }
    float L = 0.f, fw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fw[i] = mw[i] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f((mw[i] - M) * c);
      L += fw[i] * mls[256 + i * 64 + row];
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    if (tok >= 0) {
      float acc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4* src = reinterpret_cast<const f32x4*>(reinterpret_cast<float*>(ring) + i * 4096 + row * 64 + d0);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 x = src[q4];
          acc[4 * q4 + 0] += fw[i] * x[0];
          acc[4 * q4 + 1] += fw[i] * x[1];
          acc[4 * q4 + 2] += fw[i] * x[2];
          acc[4 * q4 + 3] += fw[i] * x[3];
        }
      }
      uint32_t wv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bf16x2 x = {(__bf16)(acc[2 * e] * inv), (__bf16)(acc[2 * e + 1] * inv)};
        wv[e] = __builtin_bit_cast(uint32_t, x);
      }
      u32x4* o4 = reinterpret_cast<u32x4*>(p.out + tok * p.out_stride + (int64_t)h * 64 + d0);
      o4[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
      o4[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
    }
  }
}

__global__ __launch_bounds__(256, 2) void sparse_attn_kernel(AttnParams p) {
  attn_body<false>(p, __builtin_amdgcn_workgroup_id_x());
}

// Work-group g reads the markers of items g, g + G, g + 2G, ... (G = fix_groups), 64 at a time on
// wave 0's lanes, and walks the marked ones exactly, one after the other.
__global__ __launch_bounds__(256, 2) void sparse_attn_fixup_kernel(AttnParams p) {
  __shared__ uint64_t marked;
  const int tid = __builtin_amdgcn_workitem_id_x();
  const int G = p.fix_groups;
  for (int base = __builtin_amdgcn_workgroup_id_x(); base < p.n_items; base += 64 * G) {
    if (tid < 64) {
      const int item = base + G * tid;
      bool m = false;
      if (item < p.n_items) {
        const Item d = decode_item(p, item);
        m = d.kind != kSkip && *reinterpret_cast<const volatile uint16_t*>(item_marker(p, d)) == 0xFFFFu;
      }
      const uint64_t b = __ballot(m);
      if (tid == 0) marked = b;
    }
    __syncthreads();
    uint64_t b = marked;
    b = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    __syncthreads();  // every wave has read the mask before the next batch writes it
    while (b) {
      const int l = __builtin_ctzll(b);
      b &= b - 1;
      attn_body<true>(p, base + G * l);
      __syncthreads();  // the next item reuses the LDS
    }
  }
}

// Work items of a head, in up to two segments of similar items, with the number of key-tile steps
// one item walks (its duration); the launch orders segments longest item first, so the long walks
// (dense rows, special rows of the frame patterns) do not start last and leave a tail.
struct Seg {
  int h, base, items;
  int64_t steps;
};

static int head_segments(int h, int pat, bool tokord, bool framed, int ntt, const Geom& g, int sel_width,
                         int64_t ks_cap, Seg* out) {
  const int ns4 = (g.nst + 3) / 4, groups_pf = (g.NBf + 3) / 4;
  int n = 0;
  auto add = [&](int base, int items, int64_t steps) {
    if (items > 0) out[n++] = Seg{h, base, items, steps};
  };
  if (framed) {  // four query tiles of one frame per item; one or two frames of key tiles
    add(0, g.F * ((g.NBT + 3) / 4), (int64_t)g.NBT * (pat == SAF3R_ANCHOR_LOCAL ? 2 : 1));
    return n;
  }
  switch (pat) {
    case SAF3R_DENSE:
      if (tokord) add(0, (ntt + 3) / 4, ntt);
      else add(0, (g.NT + 3) / 4, g.NT);
      break;
    case SAF3R_KEYSET: add(0, (g.NT + 3) / 4, ks_cap / 64); break;
    case SAF3R_BROADCAST: {
      const int nq = (g.T + 63) / 64;
      add(0, g.F * ((nq + 3) / 4), nq);
      break;
    }
    case SAF3R_SKIP: add(0, (g.NT + 3) / 4, 1); break;
    case SAF3R_TOKEN_DYNAMIC: add(0, ns4, g.NT); break;
    case SAF3R_TOKEN_DYNAMIC_KEYSET: add(0, ns4, ks_cap / 64); break;
    case SAF3R_BLOCK_DYNAMIC:
      add(0, ns4, g.NT);
      add(ns4, g.F * g.NBf, max(1, sel_width / 2));
      break;
    default: {  // frame-relative patterns: one special tile per item, four patch tiles per item
      const int64_t mult = pat == SAF3R_ANCHOR_LOCAL ? 2 : 1;
      const int64_t span = pat == SAF3R_ANCHOR ? 1 : (g.ns > 0 ? (64 + g.ns - 1) / g.ns + 1 : 1);
      add(0, g.nst, span * (g.NBf + 1) * mult);
      add(g.nst, g.F * groups_pf, (g.NBf + 1) * mult);
    }
  }
  return n;
}

// the K + V bytes of the block-dynamic heads above which split-mode walks are clock-paced
constexpr int64_t kSplitPacedMinBytes = (int64_t)256 << 20;

// Default step times of the key walks (the first call on a pace state, or without one), from sweeps
// at the 128-frame VGGT shape: the split value sits at the long end of the plateau of best
// block-dynamic throughput (a phase shorter than the walk's real step time scatters the work-groups
// over the key frames, a longer one costs little). Converted to wall-clock ticks with the device's
// clock rate, queried on every call (no cached state).
static void set_phase(AttnParams* p, bool fixed_order) {
  p->phase_dense = p->phase_split = 0;
  if (fixed_order) return;
  const double dense_ns = 2600.0, split_ns = 2250.0;
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
      khz <= 0)
    return;  // no wall clock: fixed order
  const double ticks_per_ns = khz * 1e-6;
  p->phase_dense = (uint64_t)fmax(1.0, dense_ns * ticks_per_ns);
  p->phase_split = (uint64_t)fmax(1.0, split_ns * ticks_per_ns);
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_sparse_attn_fwd(const void* q_packed, const void* k_packed, const void* v_packed, int frames,
                                     int tokens_per_frame, int num_special, int num_heads,
                                     const int32_t* head_pattern, const int32_t* sel, int sel_width, float scale,
                                     void* out, int64_t out_row_stride, const void* keyset_k, const void* keyset_v,
                                     const int32_t* keyset_count, int64_t keyset_capacity, const void* bcast_q,
                                     const void* bcast_k, const void* bcast_v, const uint8_t* token_order,
                                     const uint8_t* q_scaled, int flags, unsigned long long* pace,
                                     unsigned int pace_seq, void* stream) {
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
  int n_dyn = 0, n_ks = 0, n_bc = 0;
  for (int h = 0; h < num_heads; ++h) {
    int pt = head_pattern[h];
    if (pt < SAF3R_DENSE || pt > SAF3R_TOKEN_DYNAMIC_KEYSET)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: head %d has unknown pattern %d", h, pt);
    p.pattern[h] = (int8_t)pt;
    p.slot[h] = (int8_t)(pt == SAF3R_BLOCK_DYNAMIC ? n_dyn++
                         : (pt == SAF3R_KEYSET || pt == SAF3R_TOKEN_DYNAMIC_KEYSET) ? n_ks++
                         : pt == SAF3R_BROADCAST   ? n_bc++
                                                   : -1);
  }
  if (n_bc > 0) {
    if (!bcast_q || !bcast_k || !bcast_v)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: BROADCAST heads need the frame-0 and per-frame buffers");
    if (((uintptr_t)bcast_q | (uintptr_t)bcast_k | (uintptr_t)bcast_v) % 16)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: broadcast buffers must be 16-byte aligned");
  }
  p.bq = (const __bf16*)bcast_q;
  p.bk = (const __bf16*)bcast_k;
  p.bv = (const __bf16*)bcast_v;
  p.bcap = (p.g.T + 63) / 64 * 64;
  if (n_ks > 0) {
    if (!keyset_k || !keyset_v || !keyset_count)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: KEYSET heads need the compact key-set buffers");
    if (keyset_capacity <= 0 || keyset_capacity % 64)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: keyset_capacity must be a positive multiple of 64");
    if (((uintptr_t)keyset_k | (uintptr_t)keyset_v) % 16)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: key-set buffers must be 16-byte aligned");
  }
  p.kc = (const __bf16*)keyset_k;
  p.vc = (const __bf16*)keyset_v;
  p.ks_count = keyset_count;
  p.ks_cap = n_ks > 0 ? keyset_capacity : 0;
  if (n_dyn > 0) {
    if (!sel) return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: block-dynamic heads need a selection list");
    if (sel_width <= 0 || sel_width > kMaxList)
      return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: sel_width must be in [1, %d] (got %d)", kMaxList,
                  sel_width);
  }
  p.tok_order = p.framed = 0;
  if ((int64_t)frames * tokens_per_frame > 0x7fffffc0ll)
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: too many tokens");
  p.ntok = frames * tokens_per_frame;
  p.ntt = (p.ntok + 63) / 64;
  if (token_order) {
    for (int h = 0; h < num_heads; ++h) {
      const int lay = token_order[h], pt = p.pattern[h];
      if (!lay) continue;
      if (lay == SAF3R_LAYOUT_TOKEN) {
        if (pt != SAF3R_DENSE)
          return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: head %d: only DENSE heads take the token-order layout", h);
        p.tok_order |= 1ull << h;
      } else if (lay == SAF3R_LAYOUT_FRAMED) {
        if (pt != SAF3R_FRAME_LOCAL && pt != SAF3R_ANCHOR_LOCAL && pt != SAF3R_ANCHOR)
          return fail(SAF3R_ERR_INVALID,
                      "saf3r_sparse_attn_fwd: head %d: only FRAME_LOCAL / ANCHOR_LOCAL / ANCHOR heads take the framed layout", h);
        if (!framed_fits(p.g))
          return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: the framed layout does not fit this geometry");
        p.framed |= 1ull << h;
      } else {
        return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: head %d: unknown layout %d", h, lay);
      }
    }
  }
  p.q_pre = 0;
  if (q_scaled)
    for (int h = 0; h < num_heads; ++h)
      if (q_scaled[h]) p.q_pre |= 1ull << h;
  p.q = (const __bf16*)q_packed;
  p.k = (const __bf16*)k_packed;
  p.v = (const __bf16*)v_packed;
  p.sel = sel;
  p.sel_width = sel_width;
  p.out = (__bf16*)out;
  p.out_stride = out_row_stride;
  p.c = scale * 1.4426950408889634f;
  if (p.g.ns > 0 && (uint64_t)p.g.Sp * (uint64_t)p.g.ns >= 0x100000000ull)
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: too many special tokens");
  // ceil(2^32 / ns) fits 32 bits for ns >= 2 only: ns = 1 is magic 0, which the kernel tests for
  p.nsmagic = p.g.ns > 1 ? (uint32_t)((0x100000000ull + (uint64_t)p.g.ns - 1) / (uint64_t)p.g.ns) : 0u;
  if (flags & ~SAF3R_ATTN_FIXED_ORDER) return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: unknown flags 0x%x", flags);
  if ((uintptr_t)pace % 8) return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: pace must be 8-byte aligned");
  const bool fixed = (flags & SAF3R_ATTN_FIXED_ORDER) != 0;
  set_phase(&p, fixed);
  // Split-mode walks start at their first list position when the K and V rows of the block-dynamic
  // heads fit the 256 MiB Infinity Cache: work-groups that started at different times then read
  // different frames, all served from that cache, and the clock-paced order (every resident
  // work-group on the same frames) measured slower there: 16 block-top-4 heads at 32 / 48 frames
  // (185 / 278 MB) ran 548 / 725 TFLOP/s paced against 753 / 782 in that order, at 64 / 96 frames
  // (370 / 556 MB) 808 / 862 paced against 790 / 601.
  {
    int64_t split_bytes = 0;
    for (int h = 0; h < num_heads; ++h)
      if (p.pattern[h] == SAF3R_BLOCK_DYNAMIC) split_bytes += (int64_t)p.g.L * 256;  // K + V rows of 128 B
    if (split_bytes <= kSplitPacedMinBytes) p.phase_split = 0;
  }
  p.pace = fixed ? nullptr : pace;
  p.pace_read = (int)(pace_seq % 3u);
  p.pace_acc = (int)((pace_seq + 1u) % 3u);
  p.pace_zero = (int)((pace_seq + 2u) % 3u);
  Seg segs[kMaxSegs];
  int nseg = 0;
  for (int h = 0; h < num_heads; ++h)
    nseg += head_segments(h, p.pattern[h], (p.tok_order >> h) & 1, (p.framed >> h) & 1, p.ntt, p.g, sel_width,
                          keyset_capacity, segs + nseg);
  for (int i = 1; i < nseg; ++i) {  // stable: longest item first
    const Seg x = segs[i];
    int j = i;
    while (j > 0 && segs[j - 1].steps < x.steps) {
      segs[j] = segs[j - 1];
      --j;
    }
    segs[j] = x;
  }
  int64_t total = 0;
  p.n_order = nseg;
  for (int i = 0; i < nseg; ++i) {
    p.order[i] = (int16_t)segs[i].h;
    p.item_start[i] = (int)total;
    p.item_base[i] = segs[i].base;
    total += segs[i].items;
    if (total > 0x7fffffff) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: too many work items");
  }
  p.item_start[p.n_order] = (int)total;
  if (total == 0) return SAF3R_OK;
  hipLaunchKernelGGL(sparse_attn_kernel, dim3((unsigned)total), dim3(256), 0, (hipStream_t)stream, p);
  if (int e = check_launch("saf3r_sparse_attn_fwd")) return e;
  // the exact walk of the items that left the FAST range: the same items of the prescaled heads,
  // in the fixed order; every other item returns after reading its marker
  AttnParams f = p;
  f.pace = nullptr;
  f.phase_dense = f.phase_split = 0;
  int64_t ftotal = 0;
  f.n_order = 0;
  for (int i = 0; i < nseg; ++i) {
    if (!((p.q_pre >> segs[i].h) & 1) || p.pattern[segs[i].h] == SAF3R_SKIP) continue;
    f.order[f.n_order] = (int16_t)segs[i].h;
    f.item_start[f.n_order] = (int)ftotal;
    f.item_base[f.n_order] = segs[i].base;
    ftotal += segs[i].items;
    ++f.n_order;
  }
  f.item_start[f.n_order] = (int)ftotal;
  if (ftotal == 0) return SAF3R_OK;
  int cus = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  f.n_items = (int)ftotal;
  f.fix_groups = (int)std::min<int64_t>(ftotal, 2 * (int64_t)cus);  // one resident round
  hipLaunchKernelGGL(sparse_attn_fixup_kernel, dim3((unsigned)f.fix_groups), dim3(256), 0, (hipStream_t)stream, f);
  return check_launch("saf3r_sparse_attn_fwd");
}
