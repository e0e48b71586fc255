/*
 * CPU restatement of SAF3R block/token selection arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the oracle that the HIP kernels are
 * checked against. Only tests/, __graft_entry__.smoke() and the cpu_baseline leg
 * of bench.py may load it, and only to check results. The product path never calls
 * it and has no CPU fallback.
 *
 * Everything here is integer-exact or uses a fully specified fp32 operation order
 * (sequential sums, one correctly rounded division, sequential fmaf), so a GPU
 * kernel following the same order reproduces it bit for bit.
 *
 * Reference anchors (relative to the reference checkout):
 *   sortable key      saf3r/triton/topk_utils.py:26-29 (fpval_to_key)
 *   tie rule / order  saf3r/triton/fused_qk_topk.py:73-80 (composite key: sortable
 *                     fp32 bits << 32 | reversed index => ties go to the lower index),
 *                     :88-100 (flush per frame, score-descending, -1 for empty)
 *   per-frame top-k   saf3r/patch/wrapper.py:48 (topk keys *per frame*),
 *                     saf3r/triton/fused_qk_topk.py:154-160 (topk_eff = min(topk, N))
 *   block mean        saf3r/patch/adaptive_block_value.py:16-24 (mean over each block's
 *                     real population; the last block of a frame is partial)
 *
 * Parity pins (tests/test_oracle_selection.py): brute-force Python sort with an explicit
 * (key desc, index asc) order on tiny inputs; monotonicity of the key transform against
 * float comparison; -0.0 below +0.0; k >= frame size selects the whole frame; numpy
 * means for pooling; math.fsum-free fma checks against exact rational arithmetic.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* fp32 bits -> unsigned key whose integer order is the float order.
 * Negative floats (sign bit set) are bit-inverted, non-negative floats get the sign
 * bit set. -0.0 maps just below +0.0; +NaN above +inf; -NaN below -inf. */
uint32_t oracle_fkey(uint32_t bits) {
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

static uint32_t fkey_of(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return oracle_fkey(b);
}

/* bf16 bits -> fp32 (exact widening). */
static float bf16_to_f32(uint16_t h) {
    uint32_t b = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/*
 * Mean of each 64-token patch block of one head.
 * x: bf16 bits, natural token layout [F*T, D] with row stride `row_stride` (elements).
 * Frame f, patch p (0 <= p < P = T - nspec) is token f*T + nspec + p.
 * Block b of frame f covers patches [64b, min(64b+64, P)).
 * out: [F*NBf, D] fp32, row f*NBf + b. Summation order of each column (fp32 adds): the block's
 * rows in groups of ORACLE_POOL_GROUP consecutive rows; each group summed in row order from +0.0,
 * the group sums added in group order from +0.0 (a group past the population adds +0.0, which
 * changes nothing: a sum started at +0.0 is never -0.0); then one division by the population.
 * (The order is this build's definition of the block mean; the reference's mean over a block has
 * no fixed order.)
 */
#define ORACLE_POOL_GROUP 16
void oracle_block_pool(const uint16_t* x, int64_t row_stride, int F, int T, int nspec, int D,
                       int block, float* out) {
    int P = T - nspec;
    int NBf = (P + block - 1) / block;
    for (int f = 0; f < F; ++f) {
        for (int b = 0; b < NBf; ++b) {
            int p0 = b * block;
            int cnt = P - p0 < block ? P - p0 : block;
            float* o = out + ((int64_t)f * NBf + b) * D;
            for (int d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (int g0 = 0; g0 < cnt; g0 += ORACLE_POOL_GROUP) {
                    float part = 0.0f;
                    for (int r = g0; r < g0 + ORACLE_POOL_GROUP && r < cnt; ++r) {
                        int64_t tok = (int64_t)f * T + nspec + p0 + r;
                        part = part + bf16_to_f32(x[tok * row_stride + d]);
                    }
                    acc = acc + part;
                }
                o[d] = acc / (float)cnt;
            }
        }
    }
}

/* scores[i][j] = sum_d q[i][d] * k[j][d], evaluated as acc = fmaf(q, k, acc) for d = 0..D-1
 * starting from acc = 0. */
void oracle_block_scores(const float* q, const float* k, int NQ, int NK, int D, float* scores) {
    for (int i = 0; i < NQ; ++i) {
        for (int j = 0; j < NK; ++j) {
            float acc = 0.0f;
            for (int d = 0; d < D; ++d) acc = fmaf(q[(int64_t)i * D + d], k[(int64_t)j * D + d], acc);
            scores[(int64_t)i * NK + j] = acc;
        }
    }
}

/*
 * Per-frame top-k from a score matrix.
 * scores: [NQ, F*C] fp32 (C candidates per frame, candidate c of frame f at column f*C + c).
 * out:    [NQ, F*k_eff] int32, k_eff = min(k, C). For each row and frame the k_eff best
 *         candidates in order of (key(score) descending, index ascending); values are global
 *         candidate ids f*C + c. Slots beyond the candidates a frame offers stay -1 (cannot
 *         happen with k_eff = min(k, C), kept for the fixed-width layout).
 * Selection is an insertion into a sorted list with strict '>' on the key, visiting
 * candidates in increasing index: equal keys keep the earlier (lower) index ahead.
 */
int oracle_frame_topk(const float* scores, int NQ, int F, int C, int k, int32_t* out) {
    if (k <= 0 || C <= 0 || F <= 0) return -1;
    int ke = k < C ? k : C;
    uint32_t keys[1024];
    int32_t ids[1024];
    if (ke > 1024) return -2;
    for (int i = 0; i < NQ; ++i) {
        for (int f = 0; f < F; ++f) {
            const float* s = scores + (int64_t)i * F * C + (int64_t)f * C;
            int n = 0;
            for (int c = 0; c < C; ++c) {
                uint32_t key = fkey_of(s[c]);
                int pos = n;
                while (pos > 0 && key > keys[pos - 1]) --pos;
                if (pos >= ke) continue;
                int last = n < ke ? n : ke - 1;
                for (int t = last; t > pos; --t) {
                    keys[t] = keys[t - 1];
                    ids[t] = ids[t - 1];
                }
                keys[pos] = key;
                ids[pos] = f * C + c;
                if (n < ke) ++n;
            }
            int32_t* o = out + (int64_t)i * F * ke + (int64_t)f * ke;
            for (int t = 0; t < ke; ++t) o[t] = t < n ? ids[t] : -1;
        }
    }
    return 0;
}

/* Global-scope variant: the k best candidates over all F*C columns of each row
 * (same order and tie rule), width min(k, F*C). */
int oracle_global_topk(const float* scores, int NQ, int NC, int k, int32_t* out) {
    if (k <= 0 || NC <= 0) return -1;
    int ke = k < NC ? k : NC;
    uint32_t keys[1024];
    int32_t ids[1024];
    if (ke > 1024) return -2;
    for (int i = 0; i < NQ; ++i) {
        const float* s = scores + (int64_t)i * NC;
        int n = 0;
        for (int c = 0; c < NC; ++c) {
            uint32_t key = fkey_of(s[c]);
            int pos = n;
            while (pos > 0 && key > keys[pos - 1]) --pos;
            if (pos >= ke) continue;
            int last = n < ke ? n : ke - 1;
            for (int t = last; t > pos; --t) {
                keys[t] = keys[t - 1];
                ids[t] = ids[t - 1];
            }
            keys[pos] = key;
            ids[pos] = c;
            if (n < ke) ++n;
        }
        for (int t = 0; t < ke; ++t) out[(int64_t)i * ke + t] = t < n ? ids[t] : -1;
    }
    return 0;
}

/* ----------------------------------------------------------------------------------------
 * Shared key sets of the `stride` and `q_probe_topk` modes.
 *   saf3r/patch/sparse_attention.py:143-186 (q_probe_topk_attention: mean query over all
 *     tokens, scores = qbar . k / sqrt(D) in fp32, top-k keys, optional union with the
 *     anchor-frame + special indices, sorted unique key set, dense attention over it),
 *   :256-273 (stride_attention: keys start, start + stride, ..., union, unique),
 *   :56-85 (dispatch: q_probe topk = N // stride when the group has a stride, else
 *     min(topk, N); include_as defaults False for q_probe and True for stride;
 *     start = head % stride when shift is set).
 * The operation order below is the one the HIP kernels follow.
 * ---------------------------------------------------------------------------------------- */

/* Tokens per partial sum of the mean query: the N tokens split into at most 256 chunks. */
int oracle_probe_chunk(int N) { return (N + 255) / 256; }

/* Mean query of one head. q: fp32 rows in the order the mean visits them (token order, or the
 * sampled rows in list order), row stride `row_stride`.
 * For each feature: each chunk of R = oracle_probe_chunk(N) consecutive rows is summed
 * sequentially (fp32 adds, row order), the chunk sums are added sequentially in chunk
 * order, and the total is divided once by N. */
void oracle_probe_mean(const float* q, int64_t row_stride, int N, int D, float* out) {
    const int R = oracle_probe_chunk(N);
    for (int d = 0; d < D; ++d) {
        float total = 0.0f;
        for (int c0 = 0; c0 < N; c0 += R) {
            float part = 0.0f;
            const int c1 = c0 + R < N ? c0 + R : N;
            for (int t = c0; t < c1; ++t) part = part + q[(int64_t)t * row_stride + d];
            total = total + part;
        }
        out[d] = total / (float)N;
    }
}

/* Probe scores of one head: score[t] = (sequential fmaf over d of qbar[d] * k[t][d]) * scale,
 * k fp32 rows in token order, with scale = 1/sqrt(D) (a power of two for D = 64, so the product
 * is exact). */
void oracle_probe_scores(const float* qbar, const float* k, int64_t row_stride, int N, int D, float scale,
                         float* out) {
    for (int t = 0; t < N; ++t) {
        float acc = 0.0f;
        for (int d = 0; d < D; ++d) acc = fmaf(qbar[d], k[(int64_t)t * row_stride + d], acc);
        out[t] = acc * scale;
    }
}

static int cmp_u64_desc(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

/*
 * Sorted key set of one head over N = F*T tokens.
 *   mode 0 (stride): token t is in if t >= start and (t - start) % param == 0.
 *   mode 1 (top-k):  the param best tokens by (key(score) descending, index ascending),
 *                    i.e. ties go to the lower index; param >= N takes every token.
 *   include != 0:    every token of frame 0 and every special token (t % T < ns) is in.
 * out receives the member tokens in increasing order; returns their number (or < 0).
 */
int oracle_keyset(const float* scores, int N, int T, int ns, int mode, int param, int start, int include,
                  int32_t* out) {
    if (N <= 0 || T <= 0 || param <= 0 || (mode == 0 && start < 0)) return -1;
    unsigned char* in = (unsigned char*)calloc((size_t)N, 1);
    if (!in) return -2;
    if (mode == 0) {
        for (int t = start; t < N; t += param) in[t] = 1;
    } else if (mode == 1) {
        int k = param < N ? param : N;
        uint64_t* ck = (uint64_t*)malloc((size_t)N * sizeof(uint64_t));
        if (!ck) {
            free(in);
            return -2;
        }
        for (int t = 0; t < N; ++t) ck[t] = ((uint64_t)fkey_of(scores[t]) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)t);
        qsort(ck, (size_t)N, sizeof(uint64_t), cmp_u64_desc);
        for (int i = 0; i < k; ++i) in[0xFFFFFFFFu - (uint32_t)(ck[i] & 0xFFFFFFFFu)] = 1;
        free(ck);
    } else {
        free(in);
        return -1;
    }
    if (include) {
        for (int t = 0; t < N && t < T; ++t) in[t] = 1;
        for (int t = 0; t < N; ++t)
            if (t % T < ns) in[t] = 1;
    }
    int n = 0;
    for (int t = 0; t < N; ++t)
        if (in[t]) out[n++] = t;
    free(in);
    return n;
}
