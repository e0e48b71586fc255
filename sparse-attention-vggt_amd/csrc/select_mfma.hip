// Per-frame block selection of the dynamic pattern on the matrix cores, bit-identical to the
// sequential selection (block_select_frame_kernel in select.hip, the oracle's definition).
//
// ref: saf3r/triton/fused_qk_topk.py:73-100 (composite key = sortable fp32 bits << 32 | reversed
//      index, per-frame top-k, frame-major output in descending order), saf3r/patch/wrapper.py:48.
//
// Score of query block i and key block j: the sequential fmaf chain s_ij = q_i . k_j over the fp32
// block means. The kernel computes an approximation from the fp16 split records (pooled_split_row
// in common.h: x 2^s = h1 + h2 + r, |r| <= 2^-22 |x 2^s|):
//   A_ij = Q1 K1^T, then + Q1 K2^T + Q2 K1^T   (one fp32 accumulator, 12 v_mfma_f32_32x32x16_f16),
//   a_ij = A_ij 2^-(sq_i + sk_j).
// Error bound (u = 2^-24; sums taken as any order of fp32 additions with relative error <= 2u):
//   the accumulator's 192 exact fp16 products: 191 * 2^-23 (1 + 2^-10) sum|q k|; the dropped terms
//   (h2 h2', h r', r h'): 3 * 2^-22 sum|q k|; the fmaf chain of the oracle: 63 * 2^-24 sum|q k|;
//   fp16 values below the normal range: 2^-25 |q| |k|; the scaling is exact. In all less than
//   2.8e-5 |q| |k| (sum|q k| <= |q| |k|), so |a_ij - s_ij| <= E_ij = 2^-15 |q_i| |k_j| (3.05e-5).
// A (query block, frame) is certified when its k + 1 best approximate scores (by a, each carrying
// a tag in the 5 low mantissa bits that names the key: a change of at most 2^-18 |a|) are separated
// pairwise by more than thr = 2 E_max + 2^-17 |q| |k|max (E_max over the frame's key blocks): the
// exact scores then have the same order, strictly, so the top-k and its order are those of a. Every
// other pair (near ties, rows outside the bound's range: norm +inf, which makes the threshold +inf
// or NaN; a zero threshold, where the tags alone would order exact ties) is listed with its
// candidate keys: those whose tagged a is
// at least lo = (k-th best tagged a) - thr, which hold the true top-k (its members' exact scores are
// at least the k-th best's approximation minus E). Each half wave's own list of its KL best tells
// which of its keys qualify; when its last entry is at least lo, keys past it may too, and every
// key of that half is a candidate (every key of the frame when the threshold is not finite or zero).
// After its frames, the workgroup ranks the candidates of its listed pairs by their sequential fmaf
// scores and the composite key (score key, lower index first), as the oracle does (about 1.3% of
// the pairs at 128 frames on random-init weights).
//
// Decomposition: a workgroup of 4 waves owns 128 query blocks (32 per wave) of one head and a
// group of frames (or a piece of one, below). Each frame's key records (NBf rows of 256 bytes, contiguous) are copied once
// per workgroup into a 4-stage LDS ring (3 stages for 32-block frames) by LDS-DMA loads, 16-byte chunks
// XOR-swizzled by row so that the 32 rows a fragment read touches fall into 16 distinct chunk
// columns. Per frame a wave runs S^T = K . Q^T for the frame's key blocks (padded to 32 rows)
// against its 32 queries: lane (col, half) holds query col and 16 key rows 8 g + 4 half + r; each
// tagged value is inserted into a sorted list of the KL best (one max and KL - 1 med3 per value),
// the two halves exchange their lists through v_permlane32_swap and merge, and the gaps of the merged list
// decide the pair. A lane's own values carry tag v (its value index 4 g + r); entries taken from the
// other half get tag bit 4 set, so a half-0 lane reads key 8 (t & 15) / 4 + 4 (t >> 4) + (t & 3)
// back from tag t. The key scales and the frames' largest key norms are staged in LDS once per
// workgroup; the certified lists are kept in LDS and written after the frame loop, so that no
// global store sits between the ring's loads and their waits. The listed pairs wait in an LDS queue
// with room for every pair of the workgroup, and the workgroup scores their candidates exactly after
// its frames (one candidate key per thread), so the selection is one kernel and needs no workspace.
// The file is compiled without NaN semantics (no canonicalisation before max / med3): every value
// in a certified pair is finite, and finiteness itself is tested on the bits.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"

namespace saf3r {

constexpr int kSelQueue = 1024;      // LDS queue entries per workgroup: every (query block, frame) pair of it
// empty list slots and key rows past the frame: the lowest finite float, whose low mantissa bits
// are all set, so that tagging it (an OR into those bits) leaves it unchanged and never makes a NaN;
// with k <= NBf such entries never take part in a certified order
constexpr float kSelPad = -0x1.fffffep127f;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct SelMfmaParams {
  const float* mean;      // [n][2][NB][64]
  const uint16_t* split;  // [n][2][NB][2][64]
  const float* meta;      // [n][2][NB][2]
  int32_t* idx;           // [n][NB][F * ke]
  int F, NBf, NB, ke;
  int n;                  // heads
  int fpg;                // frames per frame group (at most FPW; fewer for short clips, so that
                          // all 8 XCDs get groups)
  int slots;              // work-groups per XCD in one resident round
  int pieces;             // 1: units cut into pieces (fewer units than slots)
};

// insert x into the descending list a: a[0] = max, a[t] = med3(old a[t-1], old a[t], x), every slot
// from the old list (the slots do not depend on each other)
template <int KL>
__device__ inline void list_insert(float (&a)[KL], float x) {
#pragma unroll
  for (int t = KL - 1; t > 0; --t) a[t] = __builtin_amdgcn_fmed3f(a[t - 1], a[t], x);
  a[0] = fmaxf(a[0], x);
}

// key block (within the frame) of a tagged value in a half-0 lane's merged list
__device__ inline int tag_key(float v) {
  const int t = (int)(__builtin_bit_cast(uint32_t, v) & 31u);
  return 8 * ((t & 15) >> 2) + 4 * (t >> 4) + (t & 3);
}

// LDS byte offset of 16-byte chunk c of key row r in a ring stage
__device__ inline int sel_chunk(int r, int c) { return (r * 16 + (c ^ (r & 15))) * 16; }

// KL: list length (k + 1 rounded up: 5, 9, 17); NG: groups of 8 key blocks per frame (ceil(NBf / 8)).
// FPW = 32 / (KL - 1) frames per workgroup (a workgroup's lists are staged in LDS, one byte per
// entry); at most 38 KB of LDS (four workgroups per CU). For lists of up to 9 the compiler is held
// to four waves per SIMD (at most 128 VGPRs; the exact pass's row loads would take more).
//
// Workgroup order (blockIdx.x = r + 8 i): the hardware hands workgroups to the 8 XCDs in turn, so r
// is the XCD, and XCD r takes the frame groups g = r + 8 j only. Each XCD's L2 then holds the key
// records of 1/8 of the frames (about 0.6 MB for 7 heads at 128 frames) for every query tile,
// instead of all of them. A group holds fpg = min(FPW, ceil(F / 8)) frames, so that short clips
// still give every XCD groups. Each (head, query tile, group) unit runs in one workgroup; when XCD 0
// has fewer units than the S workgroups an XCD holds at once, each unit is cut into pieces of a few
// frames so that all S slots work (a workgroup's fixed part, about 8 us of loads, list writes and
// the exact pass, makes pieces lose once the units fill a round).
template <int KL, int NG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KL <= 9 ? 4 : 1))) void block_select_mfma_kernel(
    SelMfmaParams p) {
  constexpr int FPW = 32 / (KL - 1);
  constexpr int OPB = 36;  // bytes per query row of the staged lists (9 words: no bank conflicts)
  constexpr int kStage = NG * 8 * 256;  // bytes per ring stage: 8 NG key rows of 256 bytes
  // LDS ring stages (frames): 4 (three frames in flight), 3 for 32-block frames, so that four
  // workgroups fit a CU's LDS
  constexpr int kSelRing = NG <= 3 ? 4 : 3;
  __shared__ __align__(16) char ring[kSelRing * kStage];
  // [query][frame in group * ke + t]: the key block in its frame; for a listed pair the first byte is
  // kQueued (its entry is in the queue)
  __shared__ __align__(16) uint8_t outb[128 * OPB];
  __shared__ __align__(16) float ksc[FPW][32];  // 2^-sk of the frame's key blocks (0 past NBf)
  __shared__ float nkm[FPW];                    // the frame's largest key norm bound
  // listed pairs: (query in the group << 24 | frame in the group << 16 | first candidate), candidate mask
  __shared__ u32x2 queue[kSelQueue];
  // pairs << 16 | candidates: one atomic gives a listed pair its queue slot and its candidates' offset
  __shared__ uint32_t qctr;
  static_assert(128 * FPW <= kSelQueue && FPW <= 256 && kSelQueue * 32 <= 65536,
                "the queue holds every pair of the workgroup; fields fit their bits");
  constexpr uint8_t kQueued = 0xFE;
  const int tid = tid_x(), lane = tid & 63, w = tid >> 6, col = lane & 31, half = lane >> 5;
  const int64_t NB = p.NB;
  const int G = (p.F + p.fpg - 1) / p.fpg;
  const int xr = bid_x() & 7;
  int hs, qt, g;
  uint32_t piece = 0, m = 1;  // piece of m of the unit's frames
  if (!p.pieces) {  // blockIdx = (xr + 8 (j + cm qt), 1, head), cm = ceil(G / 8): one unit each
    const int cm = (G + 7) / 8, xq = bid_x() >> 3;
    qt = xq / cm;
    g = xr + 8 * (xq - qt * cm);
    hs = bid_z();
    if (g >= G) return;  // an empty slot of the XCD order: the whole workgroup leaves
  } else {  // fewer units than slots: blockIdx.x = xr + 8 wi, XCD xr's units cut into S pieces
    // (32-bit arithmetic: the entry keeps the units of an XCD at most 2^27)
    const uint32_t nqt = (uint32_t)((NB + 127) / 128);
    const uint32_t wi = bid_x() >> 3;
    const uint32_t cnt = G > xr ? (uint32_t)(G - xr + 7) / 8u : 0u;  // frame groups of this XCD
    const uint32_t Q = (uint32_t)p.n * nqt * cnt, S = (uint32_t)p.slots;
    if (Q == 0 || wi >= S) return;
    const uint32_t base = S / Q, extra = S - base * Q;  // m = base + 1 for the first extra units
    uint32_t unit;
    if (wi < extra * (base + 1)) {
      m = base + 1;
      unit = wi / m;
      piece = wi - unit * m;
    } else {
      m = base;
      const uint32_t t2 = wi - extra * (base + 1);
      unit = extra + t2 / m;
      piece = t2 - (unit - extra) * m;
    }
    const uint32_t pr = unit / cnt;
    hs = (int)(pr / nqt);
    qt = (int)(pr - (uint32_t)hs * nqt);
    g = xr + 8 * (int)(unit - pr * cnt);
  }
  const int gnf = min(p.F - g * p.fpg, p.fpg);  // frames of group g
  const int f0 = g * p.fpg + (int)(piece * (uint32_t)gnf / m), f1 = g * p.fpg + (int)((piece + 1) * (uint32_t)gnf / m);
  if (f0 >= f1) return;  // an empty piece (more pieces than frames)
  const int nf = f1 - f0;
  const int qloc = 32 * w + col;  // query block within the workgroup
  const int64_t qi = (int64_t)qt * 128 + qloc;
  const bool qvalid = qi < NB;
  const int64_t qrec = (int64_t)hs * 2 * NB + (qvalid ? qi : NB - 1);  // tensor 0 = q
  const int64_t krec0 = ((int64_t)hs * 2 + 1) * NB;                   // tensor 1 = k

  // ring fill: every thread issues two 16-byte copies per frame (the same count in every wave, which
  // the waits below rely on): thread t copies LDS chunks (256 u + t) mod 128 NG of the stage (row =
  // chunk / 16, the global chunk through the swizzle; rows past NBf repeat the frame's last row;
  // with fewer than 512 chunks some copies repeat others, same data to the same place). 128 NG is a
  // multiple of 64, so a wave's chunks stay contiguous from its base.
  // The copies take the scalar-base form: the frame's records as a uniform base, the lane's byte
  // offset in them (foff) and the wave's LDS offset in the stage (fdst) fixed per thread.
  const uint32_t ring_base = lds_addr(ring);
  uint32_t foff[2], fdst[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int base = (256 * u + 64 * w) % (NG * 128), pos = base + lane;
    const int r = pos >> 4, c = (pos & 15) ^ (r & 15);
    const int rr = r < p.NBf ? r : p.NBf - 1;
    foff[u] = (uint32_t)(rr * 128 + 8 * c) * 2u;
    fdst[u] = __builtin_amdgcn_readfirstlane((uint32_t)(16 * base));  // uniform: base depends on the wave only
  }
  auto fill = [&](int f, int stage) {  // frame f into ring stage `stage` ((f - f0) mod kSelRing)
    const uint32_t st = ring_base + (uint32_t)(stage * kStage);
    const uint16_t* frec = p.split + (krec0 + (int64_t)f * p.NBf) * 128;  // the frame's key records
    dma16s(frec, foff[0], st + fdst[0]);
    dma16s(frec, foff[1], st + fdst[1]);
  };
  // the first frames' copies go out first, so that their latency overlaps that of the loads below
  for (int j = 0; j < kSelRing - 1; ++j)
    if (j < nf) fill(f0 + j, j);

  // Q fragments: lane (col, half) holds features 32 half + 8 st .. + 7 of its query, both fp16 parts
  f16x8 qf[2][4];
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(p.split + qrec * 128 + 32 * half);
#pragma unroll
    for (int pc = 0; pc < 2; ++pc)
#pragma unroll
      for (int st = 0; st < 4; ++st) qf[pc][st] = __builtin_bit_cast(f16x8, src[pc * 8 + st]);
  }
  const float2 qm = *reinterpret_cast<const float2*>(p.meta + qrec * 2);

  // key meta of the workgroup's frames: the scale of every key block in LDS, and the frame's largest
  // norm bound (the 32 threads of a frame's entries, a half wave, reduce it by shuffles)
  if (tid == 0) qctr = 0;
  for (int e0 = 0; e0 < FPW * 32; e0 += 256) {
    const int e = e0 + tid, fl = e >> 5, j = e & 31;
    float2 m = {0.f, 0.f};  // rows past the frame: no norm, no scale
    if (fl < nf && j < p.NBf) m = *reinterpret_cast<const float2*>(p.meta + (krec0 + (int64_t)(f0 + fl) * p.NBf + j) * 2);
    if (fl < FPW) ksc[fl][j] = m.y;
    float mx = m.x;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (j == 0 && fl < FPW) nkm[fl] = mx;
  }
  __syncthreads();

  // threshold factor in units of A 2^-sk: 2 E + the tag truncation (2^-17 |q| |k|), times 2^sq
  const float cq = (0x1p-14f + 0x1p-17f) * qm.x / qm.y;
  const int kr = col < p.NBf ? col : p.NBf - 1;  // this lane's key row
  const uint32_t all_keys = p.NBf >= 32 ? 0xFFFFFFFFu : (1u << p.NBf) - 1u;
  const uint32_t half0_keys = all_keys & 0x0F0F0F0Fu, half1_keys = all_keys & 0xF0F0F0F0u;

  // wait until frame g's copy has landed, with `after` frames issued after it still in flight (two
  // copies per frame: the loop issues no other vector memory operation)
  static_assert(kSelRing >= 3 && kSelRing <= 5, "the waits below count up to 3 frames in flight");
  auto wait_frame = [](int after) {
    switch (after) {
      case 3: wait_vm<6>(); break;
      case 2: wait_vm<4>(); break;
      case 1: wait_vm<2>(); break;
      default: wait_vm<0>(); break;
    }
  };
  // LDS byte offsets of this lane's eight fragment chunks in a stage (one register each)
  uint32_t koff[2][4];
#pragma unroll
  for (int pc = 0; pc < 2; ++pc)
#pragma unroll
    for (int st = 0; st < 4; ++st) koff[pc][st] = (uint32_t)sel_chunk(kr, 8 * pc + 4 * half + st);
  auto products = [&](int stage) {  // K fragments of the frame in ring stage `stage`, 12 matrix products
    const char* stg = ring + stage * kStage;
    f16x8 kf[2][4];
#pragma unroll
    for (int pc = 0; pc < 2; ++pc)
#pragma unroll
      for (int st = 0; st < 4; ++st) kf[pc][st] = *reinterpret_cast<const f16x8*>(stg + koff[pc][st]);
    f32x16 a = {};
#pragma unroll
    for (int st = 0; st < 4; ++st) a = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0][st], qf[0][st], a, 0, 0, 0);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      a = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0][st], qf[1][st], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[1][st], qf[0][st], a, 0, 0, 0);
    }
    return a;
  };

  // Software pipeline: the products of frame f + 1 are issued before the list work of frame f, so
  // the matrix cores run them while the same wave works through the lists.
  wait_frame(min(kSelRing - 2, f1 - 1 - f0));
  barrier_only();
  if (f0 + kSelRing - 1 < f1) fill(f0 + kSelRing - 1, kSelRing - 1);
  // one frame: its list work on acc (its products), after issuing the next frame's products. ST:
  // the frame's ring stage when the caller knows it at compile time (LDS reads then take it as an
  // immediate offset), else -1
  auto step = [&](auto stc, const int f, const f32x16& acc) -> f32x16 {
    constexpr int ST = decltype(stc)::value;
    const int fl = f - f0;
    const int stage = ST >= 0 ? ST : fl % kSelRing;
    // frame f + 1's copy landed, and every wave has read frame f's fragments (before this barrier),
    // so frame f + kSelRing may take its stage; after the last frame every copy has landed, and the
    // next stage's products run on whatever it holds (unused)
    wait_frame(min(kSelRing - 2, f1 - 2 - f));
    barrier_only();
    if (f + kSelRing < f1) fill(f + kSelRing, stage);
    const f32x16 acc_next = products(stage + 1 == kSelRing ? 0 : stage + 1);
    // this lane's key blocks 8 g + 4 half + r: their scales (one 16-byte read per group of four)
    float ks[NG][4];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(&ksc[fl][8 * g + 4 * half]);
#pragma unroll
      for (int r = 0; r < 4; ++r) ks[g][r] = x[r];
    }
    const float thr = cq * nkm[fl];
    float lst[KL];
#pragma unroll
    for (int t = 0; t < KL; ++t) lst[t] = kSelPad;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int v = 4 * g + r;
        const float av = acc[v] * ks[g][r];
        float x = __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, av) & ~31u) | (uint32_t)v);
        if (g == NG - 1) x = 8 * g + 4 * half + r < p.NBf ? x : kSelPad;  // past the frame
        list_insert<KL>(lst, x);
      }
    // merge with the other half's list (lanes l and l + 32 hold the same query): the whole partner
    // list first, then the insertions (an entry exchanged after an insertion could be one's own).
    // One v_permlane32_swap of an entry with itself leaves [own, partner's] on a half-0 lane and
    // [partner's, own] on a half-1 lane: every lane merges the second into the first, with tag bit 4
    // on the second, so a half-0 lane (the only one whose merged list is used) keeps its own list
    // and takes its partner's without a select.
    float own[KL], other[KL];  // on half-0 lanes: this half's list (its candidates) and the partner's
#pragma unroll
    for (int t = 0; t < KL; ++t) {
      const uint32_t u = __builtin_bit_cast(uint32_t, lst[t]);
      const auto rr = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      own[t] = __builtin_bit_cast(float, (uint32_t)rr[0]);
      other[t] = __builtin_bit_cast(float, (uint32_t)rr[1] | 16u);
    }
#pragma unroll
    for (int t = 0; t < KL; ++t) lst[t] = own[t];
#pragma unroll
    for (int t = 0; t < KL; ++t) list_insert<KL>(lst, other[t]);
    // certification: a finite threshold (every row in the bound's range, so every value finite) and
    // the k + 1 best pairwise separated by more than it (with ke = NBf the gap after the last is not
    // needed)
    // (a zero threshold, from a zero query or a frame of zero keys, leaves only the tags to order
    // exact ties: such pairs are listed with every key)
    const bool finite = (__builtin_bit_cast(uint32_t, thr) & 0x7F800000u) != 0x7F800000u;  // on the bits
    const bool usable = finite && thr > 0.f;
    // (every term evaluated: no branches)
    bool ok = usable;
#pragma unroll
    for (int t = 0; t < KL - 1; ++t) ok = ok & ((t >= p.ke) | (t + 1 == p.NBf) | (lst[t] - lst[t + 1] > thr));
    if (half == 0) {
      uint8_t* o = outb + qloc * OPB + fl * p.ke;
      if (ok) {
        if (p.ke == 4) {  // one aligned word (OPB and 4 fl are multiples of 4)
          *reinterpret_cast<uint32_t*>(o) = (uint32_t)tag_key(lst[0]) | ((uint32_t)tag_key(lst[1]) << 8) |
                                            ((uint32_t)tag_key(lst[2]) << 16) | ((uint32_t)tag_key(lst[3]) << 24);
        } else {
#pragma unroll
          for (int t = 0; t < KL - 1; ++t)
            if (t < p.ke) o[t] = (uint8_t)tag_key(lst[t]);
        }
      } else if (qvalid) {
        // candidates: each half's entries at least lo; every key of a half whose last entry is at
        // least lo too (keys past its list may qualify), of the frame when the threshold is not
        // finite or the whole frame is selected
        float kth = lst[0];
#pragma unroll
        for (int t = 1; t < KL; ++t)
          if (t < p.ke) kth = lst[t];
        const float lo = kth - thr;
        uint32_t mask = 0;
#pragma unroll
        for (int t = 0; t < KL; ++t) {
          if (own[t] >= lo) mask |= 1u << tag_key(own[t]);
          if (other[t] >= lo) mask |= 1u << tag_key(other[t]);
        }
        if (own[KL - 1] >= lo) mask |= half0_keys;
        if (other[KL - 1] >= lo) mask |= half1_keys;
        if (!usable || p.ke >= p.NBf) mask = all_keys;
        mask &= all_keys;
        uint32_t nc = (uint32_t)__builtin_popcount(mask);
        if (nc < (uint32_t)p.ke) {  // cannot happen (the list's best k qualify); every key, to be safe
          mask = all_keys;
          nc = (uint32_t)__builtin_popcount(mask);
        }
        const uint32_t at = atomicAdd(&qctr, (1u << 16) | nc);  // slot at >> 16, candidates from at & 0xFFFF
        queue[at >> 16] = u32x2{((uint32_t)qloc << 24) | ((uint32_t)fl << 16) | (at & 0xFFFFu), mask};
        o[0] = kQueued;
      }
    }
    return acc_next;
  };
  // four frames per trip (one per ring stage), so that the two accumulators alternate instead of
  // being copied and the stages are compile-time offsets (lists of up to 5 and at most 24 blocks
  // per frame; otherwise the second accumulator's registers spill or push scalar values out: one
  // frame per trip)
  f32x16 acc0 = products(0), acc1;
  int fs = f0;
  if constexpr (NG <= 3 && KL <= 5) {
    static_assert(kSelRing == 4, "one trip walks the four stages");
    for (; fs + 3 < f1; fs += 4) {
      acc1 = step(std::integral_constant<int, 0>{}, fs, acc0);
      acc0 = step(std::integral_constant<int, 1>{}, fs + 1, acc1);
      acc1 = step(std::integral_constant<int, 2>{}, fs + 2, acc0);
      acc0 = step(std::integral_constant<int, 3>{}, fs + 3, acc1);
    }
  }
  for (; fs < f1; ++fs) acc0 = step(std::integral_constant<int, -1>{}, fs, acc0);
  __syncthreads();
  // the certified lists: two threads per query, frames of one parity each (the listed pairs are
  // written by the exact pass below); k = 4 lists as one 16-byte store when the output is aligned
  const int64_t row = (int64_t)p.F * p.ke;
  {
    const int q = tid >> 1;
    const int64_t i = (int64_t)qt * 128 + q;
    const bool a16 = ((uintptr_t)p.idx & 15) == 0;
    if (i < NB) {
      int32_t* drow = p.idx + ((int64_t)hs * NB + i) * row;
      for (int fl = tid & 1; fl < nf; fl += 2) {
        const uint8_t* o = outb + q * OPB + fl * p.ke;
        const int fb = (f0 + fl) * p.NBf;
        int32_t* dst = drow + (int64_t)(f0 + fl) * p.ke;
        if (p.ke == 4) {
          const uint32_t wv = *reinterpret_cast<const uint32_t*>(o);
          if ((wv & 0xFFu) == kQueued) continue;
          const int v0 = fb + (int)(wv & 0xFFu), v1 = fb + (int)((wv >> 8) & 0xFFu);
          const int v2 = fb + (int)((wv >> 16) & 0xFFu), v3 = fb + (int)(wv >> 24);
          if (a16) {
            *reinterpret_cast<u32x4*>(dst) = u32x4{(uint32_t)v0, (uint32_t)v1, (uint32_t)v2, (uint32_t)v3};
          } else {
            dst[0] = v0;
            dst[1] = v1;
            dst[2] = v2;
            dst[3] = v3;
          }
        } else {
          if (o[0] == kQueued) continue;
          for (int t = 0; t < p.ke; ++t) dst[t] = fb + o[t];
        }
      }
    }
  }
  // The listed pairs of this workgroup, exactly, one candidate key per thread: each pair's candidates
  // were numbered when it was listed (its first candidate's offset in its queue entry, its count the
  // popcount of its mask), every thread computes the sequential fmaf score of one candidate from the
  // fp32 means (one round of row loads for up to 256 candidates), and a candidate's rank among its
  // pair's candidates by the composite key (higher score, then lower block) places it among the k
  // best. Pairs whose candidates exceed the LDS space run in batches. The ring is free: every copy
  // has landed and every wave has passed the barrier above.
  constexpr int kCandMax = kSelRing * kStage / 6 / 4 * 4;
  static_assert(kCandMax >= 32, "the candidates of one pair fit");
  float* csc = reinterpret_cast<float*>(ring);                          // [kCandMax] scores
  uint16_t* cid = reinterpret_cast<uint16_t*>(ring + 4 * kCandMax);     // [kCandMax] pair << 5 | key
  const uint32_t ctr = qctr, nq = ctr >> 16, ntot = ctr & 0xFFFFu;
  auto first = [&](uint32_t e) { return e < nq ? (queue[e][0] & 0xFFFFu) : ntot; };  // pair e's first candidate
  for (uint32_t p0 = 0; p0 < nq;) {  // the same trips for every thread
    // pairs p0 .. p1 - 1: the longest run from p0 whose candidates fit (one pair always does)
    const uint32_t base = first(p0);
    uint32_t lo = ntot - base <= (uint32_t)kCandMax ? nq : p0 + 1, hi = nq;  // all the rest fit: no search
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (first(mid) - base <= (uint32_t)kCandMax) lo = mid;
      else hi = mid - 1;
    }
    const uint32_t p1 = lo, nc = first(p1) - base;
    for (uint32_t e = p0 + tid; e < p1; e += 256) {
      const u32x2 ent = queue[e];
      uint32_t m = ent[1], o = (ent[0] & 0xFFFFu) - base;
      while (m) {
        cid[o++] = (uint16_t)((e << 5) | (uint32_t)__builtin_ctz(m));
        m &= m - 1;
      }
    }
    __syncthreads();
    for (uint32_t c = tid; c < nc; c += 256) {
      const uint32_t v = cid[c], j = v & 31;
      const u32x2 ent = queue[v >> 5];
      const int64_t i = (int64_t)qt * 128 + (ent[0] >> 24);
      const int f = f0 + (int)((ent[0] >> 16) & 0xFFu);
      const f32x4* qr = reinterpret_cast<const f32x4*>(p.mean + ((int64_t)hs * 2 * NB + i) * 64);
      const f32x4* kv = reinterpret_cast<const f32x4*>(p.mean + (krec0 + (int64_t)f * p.NBf + j) * 64);
      f32x4 qa[16], kb[16];  // both rows in flight at once, then the chain
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        qa[d4] = qr[d4];
        kb[d4] = kv[d4];
      }
      float a = 0.f;
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        a = __builtin_fmaf(qa[d4][0], kb[d4][0], a);
        a = __builtin_fmaf(qa[d4][1], kb[d4][1], a);
        a = __builtin_fmaf(qa[d4][2], kb[d4][2], a);
        a = __builtin_fmaf(qa[d4][3], kb[d4][3], a);
      }
      csc[c] = a;
    }
    __syncthreads();
    for (uint32_t c = tid; c < nc; c += 256) {
      const uint32_t v = cid[c], e = v >> 5, j = v & 31;
      const uint64_t key = ckey(csc[c], j);
      const u32x2 ent = queue[e];
      const uint32_t b0 = (ent[0] & 0xFFFFu) - base, b1 = b0 + (uint32_t)__builtin_popcount(ent[1]);
      int rank = 0;
      for (uint32_t c2 = b0; c2 < b1; ++c2) rank += ckey(csc[c2], cid[c2] & 31u) > key ? 1 : 0;
      if (rank < p.ke) {
        const int64_t i = (int64_t)qt * 128 + (ent[0] >> 24);
        const int f = f0 + (int)((ent[0] >> 16) & 0xFFu);
        p.idx[((int64_t)hs * NB + i) * row + (int64_t)f * p.ke + rank] = f * p.NBf + (int)j;
      }
    }
    __syncthreads();  // the next batch overwrites the candidates
    p0 = p1;
  }
}

// Split records of given fp32 pooled rows (one wave per row): the input of the matrix-core select
// for means that did not come from saf3r_pack_qkv.
__global__ __launch_bounds__(256) void pooled_prepare_kernel(const float* __restrict__ mean, int64_t rows,
                                                             uint16_t* __restrict__ split, float* __restrict__ meta) {
  const int64_t r = (int64_t)bid_x() * 4 + (tid_x() >> 6);
  if (r >= rows) return;  // a whole wave leaves; no barrier follows
  const int lane = tid_x() & 63;
  pooled_split_row(mean[r * 64 + lane], lane, split + r * 128, meta + r * 2);
}

// work-groups of the selection kernel the current device holds at once (1024 if unknown)
template <int KL, int NG>
static int64_t select_slots() {
  static std::atomic<int64_t> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  if (dev < 64) {
    const int64_t v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 0, blocks = 0;
  int64_t v = 1024;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, block_select_mfma_kernel<KL, NG>, 256, 0) == hipSuccess &&
      cus > 0 && blocks > 0)
    v = (int64_t)cus * blocks;
  if (dev < 64) cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// a workgroup per (head, query tile, frame group), or, when XCD 0 (the one with the most frame
// groups) has fewer of them than it holds workgroups at once, a workgroup per slot and piece
template <int KL, int NG>
static void launch_select_one(hipStream_t st, SelMfmaParams p, int64_t units_xcd0) {
  p.slots = (int)std::max<int64_t>(1, select_slots<KL, NG>() / 8);
  p.pieces = units_xcd0 < p.slots ? 1 : 0;
  const int64_t nqt = ((int64_t)p.NB + 127) / 128, cm = ((p.F + p.fpg - 1) / p.fpg + 7) / 8;
  const dim3 grid = p.pieces ? dim3(8u * (unsigned)p.slots) : dim3((unsigned)(8 * cm * nqt), 1u, (unsigned)p.n);
  hipLaunchKernelGGL((block_select_mfma_kernel<KL, NG>), grid, dim3(256), 0, st, p);
}

template <int KL>
static void launch_select_mfma(int ng, hipStream_t st, const SelMfmaParams& p, int64_t units_xcd0) {
  switch (ng) {
    case 1: launch_select_one<KL, 1>(st, p, units_xcd0); break;
    case 2: launch_select_one<KL, 2>(st, p, units_xcd0); break;
    case 3: launch_select_one<KL, 3>(st, p, units_xcd0); break;
    default: launch_select_one<KL, 4>(st, p, units_xcd0); break;
  }
}

// frames per workgroup of the matrix-core select for this k: 32 / (list length - 1)
static int select_fpw(int ke) { return ke <= 4 ? 8 : ke <= 8 ? 4 : 2; }

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_pooled_prepare(const float* mean, int64_t rows, uint16_t* split, float* meta, void* stream) {
  if (int e = injected("saf3r_pooled_prepare")) return e;
  if (!mean || !split || !meta || rows < 0) return fail(SAF3R_ERR_INVALID, "saf3r_pooled_prepare: bad arguments");
  if (((uintptr_t)mean | (uintptr_t)split | (uintptr_t)meta) % 16)
    return fail(SAF3R_ERR_INVALID, "saf3r_pooled_prepare: buffers must be 16-byte aligned");
  if (rows == 0) return SAF3R_OK;
  if ((rows + 3) / 4 > 0x7fffffff) return fail(SAF3R_ERR_INVALID, "saf3r_pooled_prepare: too many rows");
  hipLaunchKernelGGL(pooled_prepare_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, mean,
                     rows, split, meta);
  return check_launch("saf3r_pooled_prepare");
}

extern "C" int64_t saf3r_block_select_pooled_workspace_bytes(int n, int frames, int blocks_per_frame, int k) {
  if (n <= 0 || n > 65535 || frames <= 0 || blocks_per_frame <= 0 || blocks_per_frame > 32 ||
      (int64_t)frames * blocks_per_frame > 0x7fffffff / 64 || k < 1 || k > 32)
    return -1;
  return 0;  // every pair is taken exactly inside its workgroup; the k > 16 kernel needs none either
}

extern "C" int saf3r_block_select_pooled(const float* mean, const uint16_t* split, const float* meta, int n,
                                         int frames, int blocks_per_frame, int k, int32_t* idx, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  if (int e = injected("saf3r_block_select_pooled")) return e;
  if (!mean || !split || !meta || !idx) return fail(SAF3R_ERR_INVALID, "saf3r_block_select_pooled: null pointer");
  if (((uintptr_t)mean | (uintptr_t)split | (uintptr_t)meta) % 16)
    return fail(SAF3R_ERR_INVALID, "saf3r_block_select_pooled: pooled buffers must be 16-byte aligned");
  if (n <= 0 || n > 65535 || frames <= 0 || blocks_per_frame <= 0 ||
      (int64_t)frames * blocks_per_frame > 0x7fffffff / 64)
    return fail(SAF3R_ERR_INVALID, "saf3r_block_select_pooled: bad shape");
  if (k < 1 || k > 32) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_block_select_pooled: k must be in [1, 32] (got %d)", k);
  if (blocks_per_frame > 32)
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_block_select_pooled: at most 32 blocks per frame");
  const int NBf = blocks_per_frame, ke = k < NBf ? k : NBf;
  const int NB = frames * NBf;
  hipStream_t st = (hipStream_t)stream;
  if (ke > 16) {  // lists longer than the matrix-core path keeps: the sequential selection, head by head
    for (int h = 0; h < n; ++h) {
      const float* pq = mean + (int64_t)h * 2 * NB * 64;
      if (int rc = saf3r_block_select(pq, pq + (int64_t)NB * 64, 1, NB, frames, NBf, k, 0,
                                      idx + (int64_t)h * NB * frames * ke, stream))
        return rc;
    }
    return SAF3R_OK;
  }
  (void)workspace;  // none is needed (the size query returns 0); kept for the entry's signature
  (void)workspace_bytes;
  const int fpg = std::max(1, std::min(select_fpw(ke), (frames + 7) / 8)), groups = (frames + fpg - 1) / fpg;
  SelMfmaParams p;
  p.mean = mean;
  p.split = split;
  p.meta = meta;
  p.idx = idx;
  p.F = frames;
  p.NBf = NBf;
  p.NB = NB;
  p.ke = ke;
  p.n = n;
  p.fpg = fpg;
  p.slots = 1;
  p.pieces = 0;
  const int64_t units_xcd0 = (int64_t)n * ((NB + 127) / 128) * ((groups + 7) / 8);
  if (units_xcd0 > ((int64_t)1 << 27))  // keeps the grids and the kernel's unit arithmetic in 32 bits
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_block_select_pooled: too many (head, query tile, frame group) units");
  const int ng = (NBf + 7) / 8;
  if (ke <= 4) launch_select_mfma<5>(ng, st, p, units_xcd0);
  else if (ke <= 8) launch_select_mfma<9>(ng, st, p, units_xcd0);
  else launch_select_mfma<17>(ng, st, p, units_xcd0);
  return check_launch("saf3r_block_select_pooled");
}
