// Per-frame token top-k of q.k: the lazy selector of the reference dino_topk heads.
//
// ref: saf3r/triton/fused_qk_topk.py:26-102 (bf16 q.k with fp32 accumulation per 64-key tile;
//      composite key = sortable fp32 bits << 32 | reversed index so ties go to the lower index;
//      running per-frame top-k; frame-major flush in descending order, -1 for empty slots),
//      :120-217 (API: q [B, Nq, D], k [B, Nk, D], Nk = frames * num_toks_per_img, output
//      int32 [B, Nq, frames * min(topk, num_toks_per_img)] of key indices).
// A 256-thread workgroup owns 128 queries (32 per wave). Key tiles of 64 keys are staged in LDS,
// scored with v_mfma_f32_32x32x16_bf16 (S^T = K . Q^T); a lane holds one query and 32 keys of each
// tile, and keeps a running top-k of the keys of its half; the two lane halves of a query merge
// their lists when the frame ends. Each frame is scored twice (see token_topk_kernel).
#include <algorithm>
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
  int64_t k_fst;  // kmode 0 and 1: rows from frame f to frame f + 1 (P or frame_row_stride)
  int32_t* idx;
  // score dump (k > 16): queries q_begin .. nq - 1, score of (query qi, frame f, key j) at
  // ws[(qi - q_begin) * F * ppad + f * ppad + j], ppad = frame length rounded up to 64
  float* ws;
  int64_t q_begin;
  int ppad;
  int fgroups;  // frame groups of the selection launch (grid.y)
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

// Candidate buffer of pass 2: per lane up to kCand candidates (float bits << 32 | key index), entry i
// of thread tid at cbuf[i * 256 + tid] (a lane's entries all sit in its own bank pair: no conflicts
// whatever the fill levels), emptied into the lane's running top-K at the end of each frame. A lane
// with more candidates than that in one frame (ties on a large scale) loses the rest and has its
// frame recomputed directly at the frame's end (see token_topk_kernel).
template <int K>
constexpr int cand_cap() { return K <= 8 ? 12 : 24; }
constexpr int kStages = 3;  // K tiles in flight: the tile of step t + 2 loads while step t computes

// K-th largest of the running float list t (descending, -inf = empty) after inserting x.
template <int K>
__device__ inline void fmax_insert(float (&t)[K], float x) {
  bool c[K];
#pragma unroll
  for (int i = 0; i < K; ++i) c[i] = x > t[i];
#pragma unroll
  for (int i = K - 1; i > 0; --i) t[i] = c[i - 1] ? t[i - 1] : (c[i] ? x : t[i]);
  t[0] = c[0] ? x : t[0];
}

// Two passes per key frame over the same bf16 MFMA scores (the score of a (query, key) pair is the
// same sequence of MFMAs in both, so the same fp32 value):
//   pass 1: every lane keeps the maximum of G groups of its candidates; the K-th largest of the 2G
//           group maxima of a query (its two lane halves) is a lower bound tau of the query's K-th
//           best score in the frame (they are 2G >= K distinct candidates);
//   pass 2: only candidates with score >= tau (or unordered: a NaN never drops out) are appended to
//           the lane's LDS buffer; a candidate costs one compare and a wave-uniform branch unless
//           some lane of the wave keeps it. A lane whose buffer overflowed in the frame is served
//           at the frame's end by a direct pass of its wave over the frame's key rows in global
//           memory (same MFMAs, so the same scores) that inserts every candidate >= tau.
// A few candidates per query and frame pass (about 3 of 1369 for top-4 of N(0,1) scores), so the
// composite-key insertion that dominates a one-pass selection runs a few times per frame instead
// of for every candidate. Key tiles stream through a 3-stage LDS ring filled by LDS-DMA loads
// issued two steps ahead (rows past the frame's end load a valid row; their scores are masked).
// Step t reads its K fragments, selects over the scores of step t - 1 while those reads are in
// flight, then issues its MFMAs into the same registers; the two waves of a SIMD alternate their
// VALU and MFMA phases.
template <int K, bool FLAT, bool DUMP>
__global__ __launch_bounds__(256, K <= 8 ? 3 : 2) void token_topk_kernel(TopkParams p) {
  // groups per lane (2G >= K maxima per query): more groups give a tighter tau for larger K, so that
  // the candidates of a lane fit its buffer
  constexpr int G = K <= 4 ? 8 : 2 * K;
  __shared__ __align__(16) char ring[kStages][8192];
  constexpr int kCand = cand_cap<K>();
  __shared__ uint64_t cbuf[(kCand + 1) * 256];
  const int tid = tid_x(), lane = tid & 63, half = lane >> 5, col = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t q0 = p.q_begin + (int64_t)bid_x() * 128;
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
  // frame f: pass 1 over its tiles, then pass 2, for the frames [f_lo, f_hi) of this work-group's
  // frame group (bid_y of p.fgroups: the split only evens out the tail of the launch); DUMP: one
  // pass over frame bid_y that stores the scores (a work-group per 128 queries and frame)
  const int f_lo = __builtin_amdgcn_readfirstlane(DUMP ? bid_y() : p.F * bid_y() / p.fgroups);
  const int f_hi = __builtin_amdgcn_readfirstlane(DUMP ? f_lo + 1 : p.F * (bid_y() + 1) / p.fgroups);
  const int total = (f_hi - f_lo) * (DUMP ? 1 : 2) * tiles_pf;
  // LDS chunk position P = 256 j + 64 w + lane of a tile (instruction j of wave w) holds key row
  // P / 8, global 16-byte chunk (P % 8) ^ swz8(row): the swizzle that makes the MFMA fragment
  // reads conflict-free is applied on the load side
  int rowj[2], chj[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int P = 256 * j + 64 * w + lane;
    rowj[j] = P >> 3;
    chj[j] = (P & 7) ^ swz8(rowj[j]);
  }
  int iu = 0, ips = 0;  // tile and pass of the next step to issue
  int64_t ifr = f_lo;  // its frame
  // FLAT (kmode 0 and 1): frame f's rows are k_fst rows apart, so a tile's address is a uniform
  // base plus a fixed 32-bit lane offset (the last tile of a frame clamps its rows to the frame's
  // last row: its own offsets); otherwise every row goes through the general row mapping
  const char* kb0 = reinterpret_cast<const char*>(p.kptr + p.k_base * p.k_rs);
  const int64_t fbytes = p.k_fst * p.k_rs * 2, tbytes = 64 * p.k_rs * 2;
  uint32_t lo[2], lo_last[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    lo[j] = (uint32_t)(rowj[j] * p.k_rs * 2 + 16 * chj[j]);
    const int rl = min(64 * (tiles_pf - 1) + rowj[j], p.P - 1) - 64 * (tiles_pf - 1);
    lo_last[j] = (uint32_t)(rl * p.k_rs * 2 + 16 * chj[j]);
  }
  // the tile of sequence step `step` (the next one) into its stage; past the last step the last
  // frame's last tile is loaded again into a stage nobody reads, so every step waits on the same
  // count of loads
  // tile address of the next step to issue (FLAT), advanced by additions; stage of that step
  const char* itb = kb0 + f_lo * fbytes;
  int ist = 0;
  auto issue = [&](int step) __attribute__((always_inline)) {
    char* st = ring[ist];
    ist = ist == kStages - 1 ? 0 : ist + 1;
    if constexpr (FLAT) {
      const char* tb = itb;
      const bool last = iu == tiles_pf - 1;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        dma16s(tb, last ? lo_last[j] : lo[j], __builtin_amdgcn_readfirstlane(lds_addr(st + 4096 * j + 1024 * w)));
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int pp = min(64 * iu + rowj[j], p.P - 1);
        const __bf16* row = rows_at(p.kptr, p.k_rs, p.k_base, p.k_rpf, p.k_frs, ifr * p.P + pp);
        dma16(row + 8 * chj[j], __builtin_amdgcn_readfirstlane(lds_addr(st + 4096 * j + 1024 * w)));
      }
    }
    if (step + 1 < total) {
      itb += tbytes;
      if (++iu == tiles_pf) {
        iu = 0;
        const int adv = DUMP ? 1 : ips;
        ifr += adv;
        itb -= tiles_pf * tbytes;
        if (adv) itb += fbytes;
        ips ^= 1;
      }
    }
  };

  uint64_t a[K];  // the lane's running top-K of its half of the frame (composite keys, 0 = empty)
#pragma unroll
  for (int t = 0; t < K; ++t) a[t] = 0;
  float gmax[G];  // this lane's group maxima over the tiles of pass 1 so far
#pragma unroll
  for (int g = 0; g < G; ++g) gmax[g] = -__builtin_inff();
  float tau = -__builtin_inff();
  // LDS byte address of this lane's next entry, row n for n candidates so far in the frame (rows
  // from kCand on are written to row kCand, the spare row that absorbs writes past the buffer)
  const uint32_t wa0 = lds_addr(cbuf) + 8 * tid, wspare = wa0 + 2048 * kCand;
  uint32_t wa = wa0;
  auto count = [&]() { return (int)((wa - wa0) >> 11); };
  auto flush = [&]() __attribute__((always_inline)) {
    const int n = min(count(), kCand);
    for (int i = 0; i < n; ++i) {
      const uint64_t ent = cbuf[i * 256 + tid];
      topk_insert<K>(a, ckey(__builtin_bit_cast(float, (uint32_t)(ent >> 32)), (uint32_t)ent));
    }
    wa = wa0;
  };
  // candidate e of this lane: key 32*(e>>4) + 8*((e&15)>>2) + 4*half + (e&3) of the tile
  auto kpos = [](int e) { return 32 * (e >> 4) + 8 * ((e & 15) >> 2) + (e & 3); };
  int f = f_lo, ps = 0, u = 0;  // frame, pass and tile of the step being selected
  // Frame f again, for the lanes flagged `over`: every candidate >= tau goes straight into a[]. K
  // fragments come from global memory (this lane's rows col and 32 + col of each tile, chunks
  // 4 half .. 4 half + 3), the MFMAs run as in the main loop on the whole wave.
  auto direct = [&](bool over) __attribute__((always_inline)) {
    if (over) {
#pragma unroll
      for (int e = 0; e < K; ++e) a[e] = 0;
    }
    for (int h2 = 0; h2 < 2 * tiles_pf; ++h2) {  // 32 keys at a time: rows 32 h2 + col
      const int r = min(32 * h2 + col, p.P - 1);
      const __bf16* row;
      if constexpr (FLAT) row = reinterpret_cast<const __bf16*>(kb0 + f * fbytes) + (int64_t)r * p.k_rs;
      else row = rows_at(p.kptr, p.k_rs, p.k_base, p.k_rpf, p.k_frs, (int64_t)f * p.P + r);
      const u32x4* src = reinterpret_cast<const u32x4*>(row + 32 * half);
      bf16x8 fa[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) fa[s] = __builtin_bit_cast(bf16x8, src[s]);
      f32x16 d = {};
#pragma unroll
      for (int s = 0; s < 4; ++s) d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s], qfrag[s], d, 0, 0, 0);
      const int pb = 32 * h2 + 4 * half;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int pp = pb + kpos(e);
        if (over && !(d[e] < tau) && pp < p.P) topk_insert<K>(a, ckey(d[e], (uint32_t)pp));
      }
    }
  };
  // PADDED: the frame's last tile holds positions past the frame's end, which never count
  auto select = [&](auto padded_tag, const f32x16& s0, const f32x16& s1) __attribute__((always_inline)) {
    constexpr bool PADDED = decltype(padded_tag)::value;
    const int pbase = 64 * u + 4 * half;
    const int lim = p.P - pbase;  // candidate e is a key of the frame when kpos(e) < lim
    auto sc = [&](int e) { return e < 16 ? s0[e] : s1[e - 16]; };
    if constexpr (DUMP) {
      // keys pbase + kpos(4 i) .. + 3 are consecutive: one 16-byte store each (the rows past the
      // frame's end land in the row's padding)
      if (qvalid) {
        float* o = p.ws + (qi - p.q_begin) * ((int64_t)p.F * p.ppad) + (int64_t)f * p.ppad + pbase;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          *reinterpret_cast<f32x4*>(o + kpos(4 * i)) = f32x4{sc(4 * i), sc(4 * i + 1), sc(4 * i + 2), sc(4 * i + 3)};
      }
      if (++u == tiles_pf) {
        u = 0;
        ++f;
      }
      return;
    } else if (ps == 0) {
#pragma unroll
      for (int e = 0; e < 32; ++e)
        gmax[e % G] = fmaxf(gmax[e % G], (!PADDED || kpos(e) < lim) ? sc(e) : -__builtin_inff());
      if (u == tiles_pf - 1) {
        // K-th largest of this query's 2G group maxima (this lane's and its partner half's)
        float top[K];
#pragma unroll
        for (int i = 0; i < K; ++i) top[i] = -__builtin_inff();
#pragma unroll
        for (int g = 0; g < G; ++g) {
          uint32_t b = __builtin_bit_cast(uint32_t, gmax[g]);
          auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
          const float other = __builtin_bit_cast(float, (uint32_t)(half ? r[0] : r[1]));
          fmax_insert<K>(top, gmax[g]);
          fmax_insert<K>(top, other);
          gmax[g] = -__builtin_inff();
        }
        tau = top[K - 1];
      }
    } else {
#pragma unroll
      for (int e0 = 0; e0 < 32; e0 += 8) {
        // the wave masks of 8 candidates first, then one uniform branch each: the compares' latency
        // is paid once per 8
        uint64_t bm[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)  // >= tau, or unordered
          bm[i] = __builtin_amdgcn_ballot_w64(!(sc(e0 + i) < tau) && (!PADDED || kpos(e0 + i) < lim));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (bm[i]) {
            // every lane writes its next entry; only the lanes that keep the candidate advance (a
            // full buffer stays on the spare row)
            const int e = e0 + i;
            const bool keep = !(sc(e) < tau) && (!PADDED || kpos(e) < lim);
            const uint32_t at = min(wa, wspare);
            wa += keep ? 2048u : 0u;
            auto* ew = reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(at);
            ew[0] = (uint32_t)(pbase + kpos(e));
            ew[1] = __builtin_bit_cast(uint32_t, sc(e));
          }
        }
      }
      if (u == tiles_pf - 1) {
        // empty the buffer (or recompute an overflowed lane), merge the partner half's list, then
        // write this frame's indices
        const bool over = count() > kCand;
        if (__builtin_amdgcn_ballot_w64(over)) direct(over);
        if (over) wa = wa0;
        flush();
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
        tau = -__builtin_inff();
      }
    }
    if (++u == tiles_pf) {
      u = 0;
      if (ps) ++f;
      ps ^= 1;
    }
  };

  wait_vm<0>();  // q fragments landed; from here vmcnt counts ring loads only
  for (int s = 0; s < kStages - 1; ++s) issue(s);
  f32x16 s0 = {}, s1 = {};  // scores of the previous step
  int rst = 0;  // stage of step t
  for (int t = 0; t <= total; ++t) {
    bf16x8 ka[4], kbf[4];
    if (t < total) {
      wait_vm<2 * (kStages - 2)>();  // tile t landed: only the loads of step t + 1 are pending
      barrier_only();                // every wave's share of tile t is in LDS; every wave is done with tile t-1
      issue(t + kStages - 1);
      const char* kb = ring[rst];
      rst = rst == kStages - 1 ? 0 : rst + 1;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int chn = 4 * half + s;
        const int r0 = col, r1 = 32 + col;
        ka[s] = *reinterpret_cast<const bf16x8*>(&kb[r0 * 128 + ((chn ^ swz8(r0)) << 4)]);
        kbf[s] = *reinterpret_cast<const bf16x8*>(&kb[r1 * 128 + ((chn ^ swz8(r1)) << 4)]);
      }
    }
    if (t > 0) {
      if (64 * u + 64 > p.P) select(std::true_type{}, s0, s1);
      else select(std::false_type{}, s0, s1);
    }
    if (t < total) {
      // S^T = K . Q^T over the staged tile: keys 0..31 in s0, 32..63 in s1
      s0 = f32x16{};
      s1 = f32x16{};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[s], qfrag[s], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kbf[s], qfrag[s], s1, 0, 0, 0);
      }
    }
  }
  wait_vm<0>();  // the trailing loads into unread stages land before the work-group's LDS is released
}

template <int K>
static int launch_topk(TopkParams p, hipStream_t st) {
  // Frame groups: every work-group walks all frames of its queries in 2 passes, so with few, long
  // work-groups the launch ends with a partly idle last round. The frames split into g groups (one
  // work-group per 128 queries and group): the largest g of at most 16, with at least 8 frames a
  // group, whose rounds of resident work-groups (K <= 8: 3 per CU, else 2) are within 2% of the
  // fullest (at 128 frames x 1369 tokens: g = 16, 10.5 ms against 10.9 with g = 5 and 13.2 with
  // one group).
  const int64_t nb = (p.nq + 127) / 128;
  int cus = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int64_t slots = (int64_t)cus * (K <= 8 ? 3 : 2);
  const int gmax = std::max(1, std::min(16, p.F / 8));
  auto eff = [&](int g) {
    const int64_t wgs = nb * g, rounds = (wgs + slots - 1) / slots;
    return (double)wgs / (double)(rounds * slots);
  };
  double best_eff = 0.0;
  for (int g = 1; g <= gmax; ++g) best_eff = std::max(best_eff, eff(g));
  int best = 1;
  for (int g = gmax; g >= 1; --g)
    if (eff(g) >= best_eff - 0.02) {
      best = g;
      break;
    }
  p.fgroups = best;
  const dim3 grid((unsigned)nb, (unsigned)best);
  if (p.kmode == 2) hipLaunchKernelGGL((token_topk_kernel<K, false, false>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((token_topk_kernel<K, true, false>), grid, dim3(256), 0, st, p);
  return check_launch("saf3r_token_topk");
}

// ---- per-frame top-k for 16 < k <= 128 (the reference's range): scores, then a selection ----
constexpr int kLargeMaxP = 4096;  // frame length of that path (values of a segment held by one wave)

// One wave per (query row, frame) segment of P <= 64 NV stored scores. The ke-th largest composite
// key (sortable float key << 32 | reversed index, the order of the reference's fused top-k) is
// found by a radix select over the float keys, eight 4-bit digits from the top: every lane counts
// its own keys into its own 16 LDS bins (bin b of lane l at word 64 b + l: no two lanes share a
// bank or a word, so the adds never contend), then the wave sums each bin and picks the digit.
// Keys above the threshold value all count, keys equal to it count from the lowest index on. Each
// selected key's position is the number of selected keys above it.
template <int NV>
__global__ __launch_bounds__(256) void topk_large_kernel(const float* __restrict__ ws, int64_t q_begin, int64_t q_end,
                                                          int F, int P, int ppad, int ke, int32_t* __restrict__ idx) {
  __shared__ uint32_t hist[4][16 * 64];
  __shared__ uint64_t sel[4][128];
  const int lane = tid_x() & 63, w = tid_x() >> 6;
  const int64_t seg = (int64_t)bid_x() * 4 + w;
  if (seg >= (q_end - q_begin) * F) return;  // a whole wave leaves; no work-group barrier follows
  const int64_t r = seg / F;
  const int f = (int)(seg - r * F);
  const float* src = ws + r * ((int64_t)F * ppad) + (int64_t)f * ppad;
  uint32_t key[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = lane + 64 * i;
    key[i] = j < P ? fkey(src[j]) : 0;
  }
  uint32_t* hw = hist[w];
  uint32_t prefix = 0, mask = 0;
  int need = ke;  // keys still to take at or below the current prefix
  const int b = lane & 15, g = lane >> 4;  // the bin this lane sums, and its quarter of the lanes
#pragma unroll 1
  for (int sh = 28; sh >= 0; sh -= 4) {
#pragma unroll
    for (int t = 0; t < 16; ++t) hw[64 * t + lane] = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (lane + 64 * i < P && (key[i] & mask) == prefix) atomicAdd(&hw[64 * ((key[i] >> sh) & 15) + lane], 1u);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this lane's counts are in
    __builtin_amdgcn_wave_barrier();
    // total of bin b: lanes 16 g .. 16 g + 15 here, the other quarters through two exchanges
    const u32x4* hb = reinterpret_cast<const u32x4*>(hw + 64 * b + 16 * g);
    uint32_t tot = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 x = hb[t];
      tot += x[0] + x[1] + x[2] + x[3];
    }
    tot += __shfl_xor(tot, 16);
    tot += __shfl_xor(tot, 32);
    // keys in bins above b (lanes b + 1 .. 15 of the first quarter hold them)
    uint32_t incl = tot;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const uint32_t y = __shfl_down(incl, o, 16);
      if (b + o < 16) incl += y;
    }
    const uint32_t above = incl - tot;
    const bool hit = lane < 16 && above < (uint32_t)need && (uint32_t)need <= incl;
    const uint64_t m = __ballot(hit);
    const int src_lane = (int)__builtin_ctzll(m);
    const int digit = __shfl(b, src_lane);
    need -= (int)__shfl(above, src_lane);
    prefix |= (uint32_t)digit << sh;
    mask |= 0xFu << sh;
    __builtin_amdgcn_wave_barrier();
  }
  // selected: keys above the threshold value, and the first `need` keys equal to it, by index
  int cnt = 0, eqseen = 0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = lane + 64 * i;
    const bool valid = j < P;
    const bool gt = valid && key[i] > prefix, eq = valid && key[i] == prefix;
    const uint64_t meq = __ballot(eq);
    const int req = eqseen + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(meq >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)meq, 0));
    const bool take = gt || (eq && req < need);
    const uint64_t mt = __ballot(take);
    const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mt >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mt, 0));
    if (take) sel[w][pos] = ((uint64_t)key[i] << 32) | (uint64_t)(0xFFFFFFFEu - (uint32_t)j);
    cnt += __popcll(mt);
    eqseen += __popcll(meq);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  int32_t* o = idx + (q_begin + r) * ((int64_t)F * ke) + (int64_t)f * ke;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = lane + 64 * h;
    if (e < ke) {
      const uint64_t x = sel[w][e];
      int rank = 0;
      for (int t = 0; t < ke; ++t) rank += sel[w][t] > x;
      o[rank] = f * P + (int)ckey_index(x);
    }
  }
}

// Bytes of one query's stored scores (frames x frame length rounded up to 64, fp32).
static int64_t large_row_bytes(int frames, int per_frame) { return (int64_t)frames * (64 * ((per_frame + 63) / 64)) * 4; }

// Queries per chunk: a workspace of at most 1 GiB in whole work-groups of 128 queries (at least one).
static int64_t large_chunk_rows(int n_q, int frames, int per_frame) {
  int64_t nqc = ((int64_t)1 << 30) / large_row_bytes(frames, per_frame) / 128 * 128;
  if (nqc < 128) nqc = 128;
  const int64_t nq128 = ((int64_t)n_q + 127) / 128 * 128;
  return nqc < nq128 ? nqc : nq128;
}

// The caller's workspace holds the scores of `nqc` queries at a time (whole work-groups of 128);
// chunks run one after another on the stream, so one workspace serves every chunk.
static int token_topk_large(TopkParams p, int n_q, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  const int tiles = (p.P + 63) / 64;
  p.ppad = 64 * tiles;
  const int64_t row_bytes = large_row_bytes(p.F, p.P);
  int64_t nqc = workspace_bytes / row_bytes / 128 * 128;
  if (!workspace || nqc < 128)
    return fail(SAF3R_ERR_INVALID,
                "saf3r_token_topk: min(topk, per_frame) > 16 needs a workspace of at least %lld bytes "
                "(saf3r_token_topk_workspace_bytes), got %lld",
                (long long)(128 * row_bytes), (long long)(workspace ? workspace_bytes : 0));
  if (nqc > n_q) nqc = n_q;
  p.ws = static_cast<float*>(workspace);
  const int nv = tiles <= 4 ? 4 : tiles <= 8 ? 8 : tiles <= 12 ? 12 : tiles <= 16 ? 16 : tiles <= 24 ? 24
                 : tiles <= 32 ? 32 : tiles <= 48 ? 48 : 64;
  for (int64_t q0 = 0; q0 < n_q; q0 += nqc) {
    const int64_t q1 = q0 + nqc < n_q ? q0 + nqc : n_q;
    p.q_begin = q0;
    p.nq = (int)q1;
    const dim3 g1((unsigned)((q1 - q0 + 127) / 128), (unsigned)p.F);
    if (p.kmode == 2) hipLaunchKernelGGL((token_topk_kernel<1, false, true>), g1, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((token_topk_kernel<1, true, true>), g1, dim3(256), 0, st, p);
    if (int rc = check_launch("saf3r_token_topk")) return rc;
    const dim3 g2((unsigned)(((q1 - q0) * p.F + 3) / 4));
    switch (nv) {
      case 4: hipLaunchKernelGGL(topk_large_kernel<4>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      case 8: hipLaunchKernelGGL(topk_large_kernel<8>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      case 12: hipLaunchKernelGGL(topk_large_kernel<12>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      case 16: hipLaunchKernelGGL(topk_large_kernel<16>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      case 24: hipLaunchKernelGGL(topk_large_kernel<24>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      case 32: hipLaunchKernelGGL(topk_large_kernel<32>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      case 48: hipLaunchKernelGGL(topk_large_kernel<48>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
      default: hipLaunchKernelGGL(topk_large_kernel<64>, g2, dim3(256), 0, st, p.ws, q0, q1, p.F, p.P, p.ppad, p.ke, p.idx); break;
    }
    if (int rc = check_launch("saf3r_token_topk")) return rc;
  }
  return SAF3R_OK;
}

}  // namespace saf3r

using namespace saf3r;

// Shape checks shared by saf3r_token_topk and its workspace query.
static int topk_shape(const char* who, int n_q, int frames, int per_frame, int topk) {
  if (n_q < 0 || frames <= 0 || per_frame <= 0) return fail(SAF3R_ERR_INVALID, "%s: bad shape", who);
  if (topk < 1) return fail(SAF3R_ERR_INVALID, "%s: topk must be >= 1", who);
  const int ke = topk < per_frame ? topk : per_frame;
  if (ke > 128) return fail(SAF3R_ERR_UNSUPPORTED, "%s: min(topk, per_frame) must be <= 128 (got %d)", who, ke);
  if (ke > 16 && (per_frame > kLargeMaxP || frames > 65535))
    return fail(SAF3R_ERR_UNSUPPORTED, "%s: topk > 16 needs per_frame <= %d and frames <= 65535", who, kLargeMaxP);
  return SAF3R_OK;
}

extern "C" int64_t saf3r_token_topk_workspace_bytes(int n_q, int frames, int per_frame, int topk) {
  if (topk_shape("saf3r_token_topk_workspace_bytes", n_q, frames, per_frame, topk)) return -1;
  const int ke = topk < per_frame ? topk : per_frame;
  if (ke <= 16 || n_q == 0) return 0;
  return large_chunk_rows(n_q, frames, per_frame) * large_row_bytes(frames, per_frame);
}

extern "C" int saf3r_token_topk(const saf3r_rows* q, const saf3r_rows* k, int n_q, int frames, int per_frame,
                                int topk, int32_t* idx, void* workspace, int64_t workspace_bytes, void* stream) {
  if (int e = injected("saf3r_token_topk")) return e;
  if (!q || !k || !q->ptr || !k->ptr || !idx) return fail(SAF3R_ERR_INVALID, "saf3r_token_topk: null pointer");
  if (int e = topk_shape("saf3r_token_topk", n_q, frames, per_frame, topk)) return e;
  const int ke = topk < per_frame ? topk : per_frame;
  if (workspace_bytes < 0) return fail(SAF3R_ERR_INVALID, "saf3r_token_topk: negative workspace size");
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
  p.k_fst = p.kmode == 1 ? k->frame_row_stride : per_frame;
  // the flat form addresses a frame's rows with 32-bit lane offsets from a tile base
  if (p.kmode != 2 && ((int64_t)per_frame + 64) * k->row_stride * 2 >= ((int64_t)1 << 31)) p.kmode = 2;
  p.nq = n_q;
  p.F = frames;
  p.P = per_frame;
  p.ke = ke;
  p.idx = idx;
  p.ws = nullptr;
  p.q_begin = 0;
  p.ppad = 0;
  p.fgroups = 1;
  hipStream_t st = (hipStream_t)stream;
  if (ke > 16) return token_topk_large(p, n_q, workspace, workspace_bytes, st);
  if (p.ke <= 1) return launch_topk<1>(p, st);
  if (p.ke <= 2) return launch_topk<2>(p, st);
  if (p.ke <= 4) return launch_topk<4>(p, st);
  if (p.ke <= 8) return launch_topk<8>(p, st);
  return launch_topk<16>(p, st);
}
