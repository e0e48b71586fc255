/*
 * saf3r_hip.h — C ABI of the MI355X (gfx950) kernels for SAF3R head-wise sparse global
 * attention in VGGT-style alternating frame/global transformers.
 *
 * Conventions
 *   - Every entry returns an int status (SAF3R_OK = 0). On failure nothing is launched and
 *     saf3r_last_error() returns a message (thread-local). No C++ exception crosses the ABI.
 *   - Every device buffer, workspaces included, is allocated by the caller (entries that need a
 *     workspace have a size query); the library never allocates or frees device memory and keeps
 *     no device state (the one exception is the static workspace of saf3r_probe_scores_noalloc, a
 *     device array of the library's code object). `stream` is a hipStream_t (NULL = default
 *     stream); every entry is asynchronous on it and performs no host synchronisation.
 *   - bf16 buffers are passed as void* (IEEE bfloat16, 2 bytes per element).
 *   - Host-side arrays (head tables, frequency tables) are read during the call only.
 *
 * Geometry (one global-attention layer, batch 1)
 *   F frames of T tokens: the first `num_special` tokens of each frame are special (camera +
 *   registers), the remaining P = T - num_special are patch tokens; N = F*T. head_dim = 64,
 *   block = 64. Patch tokens of a frame form NBf = ceil(P/64) blocks (the last may be partial);
 *   block b of frame f has the global block id f*NBf + b.
 *
 * Packed layout (written by saf3r_pack_qkv, read by the attention / pooling / selection kernels)
 *   Slots per head: L = Sp + F*Pp with S = F*num_special special slots first (slot s holds token
 *   (s / num_special)*T + s % num_special), padded to Sp = roundup(S, 64); then frame f's patch
 *   p at slot Sp + f*Pp + p, Pp = NBf*64. Padding slots hold zeros.
 *   Q, K: [H][L][64] bf16, rows of 128 bytes.
 *   V:    [H][L/64][64][64] bf16, one transposed 64x64 tile per 64 slots:
 *         tile[i][c] = V[slot = 64*tile + kappa(c)][d = 32*(i/32) + phi(i%32)], where
 *         kappa(c) swaps bits 2 and 3 of c, and phi(i) = 16*((i>>2)&1) + 4*(i>>3) + (i&3).
 *         (These permutations match the register layout of the MFMA 32x32x16 bf16 operands so
 *         that every LDS read in the attention kernel is a 16-byte vector.)
 *
 * Per-head layout variants (saf3r_layout, chosen per head by the token_order flags of saf3r_pack_qkv and
 * saf3r_sparse_attn_fwd; the same Q, K, V buffers and tile formats):
 *   SAF3R_LAYOUT_TOKEN  (DENSE heads): slot t holds token t (t < F*T), no special or per-frame padding.
 *   SAF3R_LAYOUT_FRAMED (FRAME_LOCAL, ANCHOR_LOCAL, ANCHOR heads): with NBT = ceil(T/64), frame f's T
 *         tokens, special ones included, in token order at slots f*NBT*64 .. f*NBT*64 + T - 1, zeros in
 *         the rest of its NBT tiles. Needs F*NBT*64 <= L, true when the special tokens fit the padding
 *         of the frame's last patch tile (NBT == NBf) or num_special == 0; every key set of these
 *         patterns is then whole frames, walked with prefix masks only.
 */
#ifndef SAF3R_HIP_H
#define SAF3R_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAF3R_ABI_VERSION 13

enum saf3r_status {
  SAF3R_OK = 0,
  SAF3R_ERR_INVALID = 1,      /* bad argument, shape or pointer */
  SAF3R_ERR_UNSUPPORTED = 2,  /* valid request this library does not implement (e.g. head_dim != 64) */
  SAF3R_ERR_LAUNCH = 3,       /* the HIP runtime rejected a launch */
  SAF3R_ERR_INJECTED = 4      /* failure forced through SAF3R_FAULT_INJECT (tests of error paths) */
};

/* Per-head attention pattern ids. Masks are given for query token i and key token j. */
enum saf3r_pattern {
  SAF3R_DENSE = 0,         /* every key.                          ref: saf3r/patch/wrapper.py:99-100 (mode "full") */
  SAF3R_FRAME_LOCAL = 1,   /* frame(j) == frame(i).               ref: saf3r/patch/sparse_attention.py:234-253 (global_to_frame) */
  SAF3R_ANCHOR_LOCAL = 2,  /* frame(j) in {0, frame(i)}.          ref: union of sparse_attention.py:134-140 and :234-253 */
  SAF3R_BLOCK_DYNAMIC = 3, /* special i: every key; patch i: patch keys of the blocks listed for
                              block(i) in the selection list.     ref: block analogue of sparse_attention.py:189-231 */
  SAF3R_TOKEN_DYNAMIC = 4, /* reference dino_topk: special rows attend every key (this entry);
                              patch rows go through saf3r_gather_attn_fwd.  ref: sparse_attention.py:189-231 */
  SAF3R_ANCHOR = 5,        /* frame(j) == 0.                      ref: sparse_attention.py:134-140 (all_to_first) */
  SAF3R_SKIP = 6,          /* output zero.                        ref: sparse_attention.py:40-41 */
  SAF3R_KEYSET = 7,        /* j in the head's shared key set (saf3r_keyset_build / _gather).
                              ref: sparse_attention.py:256-273 (stride), :143-186 (q_probe_topk) */
  SAF3R_BROADCAST = 8,     /* frame 0's attention map applied to every frame: the row of token
                              f*T + i is sum_j softmax_j(q[i] . k[j] * scale) v[f*T + j], i, j < T.
                              ref: sparse_attention.py:110-131 (broadcast_first) */
  SAF3R_TOKEN_DYNAMIC_KEYSET = 9 /* dino_topk with dino_sp2sp_stride s != 1: special rows attend the
                              head's key set (keys 0, s, 2s, ...: a SAF3R_KEYSET_STRIDE set with start 0
                              and no include), served from the key-set buffers like a KEYSET head;
                              patch rows go through saf3r_gather_attn_fwd. ref: sparse_attention.py:197-208 */
};

/* Per-head layouts of the token_order arrays (see "Per-head layout variants" above). */
enum saf3r_layout {
  SAF3R_LAYOUT_PACKED = 0, /* the packed layout */
  SAF3R_LAYOUT_TOKEN = 1,  /* token order, DENSE heads */
  SAF3R_LAYOUT_FRAMED = 2  /* frame-padded token order, FRAME_LOCAL / ANCHOR_LOCAL / ANCHOR heads */
};

/* Flags of saf3r_sparse_attn_fwd. */
enum saf3r_attn_flags {
  SAF3R_ATTN_FIXED_ORDER = 1 /* every key walk starts at its first tile: run-to-run identical output */
};

/* dtype_flags of saf3r_gather_attn_fwd: rows are bf16 unless flagged fp32. */
enum saf3r_gather_dtype {
  SAF3R_GATHER_QK_FP32 = 1, /* q and k rows are fp32 */
  SAF3R_GATHER_V_FP32 = 2,  /* v rows are fp32 */
  SAF3R_GATHER_OUT_FP32 = 4 /* out rows are fp32 (the accumulator itself, not rounded) */
};

/* Key-set kinds of saf3r_keyset_build. */
enum saf3r_keyset_mode {
  SAF3R_KEYSET_STRIDE = 0, /* tokens start, start + stride, ...      ref: sparse_attention.py:256-273 */
  SAF3R_KEYSET_TOPK = 1    /* the k best probe scores, ties to the lower token. ref: :143-186 */
};

/* Row addressing of a token-row buffer: logical row r lives at
 *   ptr + (base_row + (r / rows_per_frame) * frame_row_stride + r % rows_per_frame) * row_stride
 * elements. A plain [n, 64] matrix is {ptr, 64, 0, n, 0}. */
typedef struct saf3r_rows {
  const void* ptr;
  int64_t row_stride;
  int64_t base_row;
  int64_t rows_per_frame;
  int64_t frame_row_stride;
} saf3r_rows;

int saf3r_abi_version(void);
const char* saf3r_last_error(void);

/* Number of packed slots per head (L above). Returns -1 for an invalid geometry. */
int64_t saf3r_packed_slots(int frames, int tokens_per_frame, int num_special);

/*
 * Prologue of the patched global attention: per-head QK-LayerNorm(64) and 2-D RoPE in fp32,
 * then bf16 packing into the layout above.
 *   q, k, v: bf16, element (token t, head h, d) at ptr[t*tok_stride + h*head_stride + d]
 *            (the qkv Linear output [N, 3*H*64] is q = base, k = base + H*64, v = base + 2*H*64,
 *            tok_stride = 3*H*64, head_stride = 64).
 *   ln_*:    fp32 [64] device arrays (weight, bias), used when apply_ln != 0.
 *   pos:     int32 [N][2] device (y, x) positions, used when rope_cos != NULL.
 *   rope_cos, rope_sin: device fp32 [rope_positions][16] tables, cos / sin of
 *            position * inv_freq[i] (inv_freq[i] = 1 / base^(2i/32)); NULL disables RoPE.
 *            Positions are clamped to [0, rope_positions - 1].
 *   token_order: host uint8 [num_heads] or NULL: saf3r_layout per head (heads h < 64 only; 0 =
 *            packed). SAF3R_LAYOUT_TOKEN packs slot t = token t, SAF3R_LAYOUT_FRAMED frame f's tokens
 *            at tile f*ceil(T/64) (SAF3R_ERR_UNSUPPORTED where it does not fit): the layouts
 *            saf3r_sparse_attn_fwd reads for heads flagged the same way.
 *   fp32_heads: host uint8 [num_heads] or NULL. Heads h < 64 flagged here also get their fp32 q and k
 *            (after LayerNorm and RoPE, before the bf16 rounding) in qk32: the s-th flagged head (in
 *            increasing head order) at qk32[((s*2 + 0|1) * F*T + t) * 64 + d] for q|k of token t.
 *            (Under autocast the reference keeps q/k in fp32 after LayerNorm/RoPE; its q_probe_topk
 *            mean / scores and its dino_topk gather read those fp32 values.)
 *   q_scaled, q_scale: host uint8 [num_heads] or NULL, and a factor. The packed Q of a head h < 64
 *            flagged here is q * q_scale (fp32, after LayerNorm and RoPE), rounded once to bf16;
 *            its qk32 rows stay unscaled. With q_scale = softmax scale * log2(e) this is the
 *            prescaled Q that saf3r_sparse_attn_fwd takes for heads flagged in its q_scaled.
 *   pool_heads, pool_mean, pool_split, pool_meta: host uint8 [num_heads] or NULL, and device buffers.
 *            Heads h < 64 flagged here (packed layout only) also get the pooled block records of
 *            saf3r_block_select_pooled, for the s-th flagged head (increasing head order), tensor
 *            t = 0 (q) / 1 (k) and patch block b = f*NBf + j at record r = (s*2 + t)*F*NBf + b:
 *              pool_mean[r*64 + d]:  the block mean of bf16(q) (q after LayerNorm and RoPE, without
 *                                    q_scale) or of the packed bf16 k, summed and divided as
 *                                    saf3r_block_pool does (bit-identical to it on unscaled rows);
 *              pool_split[r*128 ...]: fp16 bits of the mean's two-part split (saf3r_pooled_prepare);
 *              pool_meta[r*2 ...]:    its norm bound and scale (saf3r_pooled_prepare).
 * Replaces: saf3r/patch/patch_vggt.py:577-583 (qkv reshape, q_norm/k_norm, rope) and
 *           saf3r/models/official_vggt/layers/rope.py:154-188.
 */
int saf3r_pack_qkv(const void* q, const void* k, const void* v, int64_t tok_stride, int64_t head_stride,
                   int frames, int tokens_per_frame, int num_special, int num_heads,
                   const float* q_ln_weight, const float* q_ln_bias, const float* k_ln_weight,
                   const float* k_ln_bias, float ln_eps, int apply_ln,
                   const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_positions,
                   void* q_packed, void* k_packed, void* v_packed, const uint8_t* token_order,
                   const uint8_t* fp32_heads, float* qk32, const uint8_t* q_scaled, float q_scale,
                   const uint8_t* pool_heads, float* pool_mean, uint16_t* pool_split, float* pool_meta,
                   void* stream);

/*
 * Pooled patch-block means (fp32) of the packed Q and K of the listed heads.
 *   head_ids: host int32 [n_heads_sel]; pooled_q / pooled_k: [n_heads_sel][F*NBf][64].
 *   k_packed / pooled_k may both be NULL (pool Q only).
 * Each column is summed in fp32 in a fixed order: the block's patch tokens in groups of 16
 * consecutive rows, each group in row order from +0.0, the group sums in group order from +0.0; then
 * one division by the block population. Results are bit-identical to that definition.
 * Replaces: block pooling of the dynamic pattern (reference precedent
 *           saf3r/patch/adaptive_block_value.py:16-24).
 */
int saf3r_block_pool(const void* q_packed, const void* k_packed, int frames, int tokens_per_frame,
                     int num_special, int num_heads, const int32_t* head_ids, int n_heads_sel,
                     float* pooled_q, float* pooled_k, void* stream);

/*
 * Per-frame top-k from fp32 scores (bit-exact entry).
 *   scores: [n][rows][frames*cands_per_frame]; idx: int32 [n][rows][frames*min(k, cands_per_frame)].
 *   For each row and frame: the min(k, C) best candidates by the sortable fp32 key, descending,
 *   ties to the lower index; values are global candidate ids f*C + c. 1 <= k <= 32.
 * Replaces: the selection of saf3r/triton/fused_qk_topk.py:73-100 (composite key, frame-major
 *           flush) applied to a given score matrix.
 */
int saf3r_topk_from_scores(const float* scores, int n, int rows, int frames, int cands_per_frame, int k,
                           int32_t* idx, void* stream);

/*
 * Block selection of the BLOCK_DYNAMIC pattern from pooled Q/K.
 *   pooled_q: [n][NBq][64]; pooled_k: [n][frames*blocks_per_frame][64] (fp32).
 *   score(i, j) = sequential fmaf over d = 0..63 starting from 0.
 *   scope 0 (per frame): idx [n][NBq][frames*min(k, NBf)], frame-major;
 *   scope 1 (global):    idx [n][NBq][min(k, frames*NBf)].
 *   Order: score key descending, ties to the lower block id. 1 <= k <= 32.
 * Replaces: the block top-k of the dynamic pattern (no reference symbol; per-frame semantics of
 *           saf3r/patch/wrapper.py:48 and saf3r/triton/fused_qk_topk.py:120-217 at block level).
 */
int saf3r_block_select(const float* pooled_q, const float* pooled_k, int n, int nbq, int frames,
                       int blocks_per_frame, int k, int scope, int32_t* idx, void* stream);

/*
 * Split records of pooled rows for saf3r_block_select_pooled, from fp32 rows mean [rows][64]:
 *   split[r*128 + d], split[r*128 + 64 + d]: fp16 bits of h1 = fp16(x * 2^s) and
 *     h2 = fp16(x * 2^s - h1), x = mean[r*64 + d], s chosen so that the row's largest magnitude times
 *     2^s lies in [2^14, 2^15) (s = 0 for a zero row);
 *   meta[r*2]: an upper bound of the row's L2 norm, or +inf when the row has a non-finite value or a
 *     largest magnitude outside [2^-50, 2^50] (such rows are always scored exactly);
 *   meta[r*2 + 1]: 2^-s.
 * No counterpart in the reference.
 */
int saf3r_pooled_prepare(const float* mean, int64_t rows, uint16_t* split, float* meta, void* stream);

/*
 * Per-frame block selection of the BLOCK_DYNAMIC pattern on the matrix cores, bit-identical to
 * saf3r_block_select (scope 0) on the same means.
 *   mean / split / meta: the pooled records of n heads (saf3r_pack_qkv pool_* or saf3r_pooled_prepare):
 *     record (s*2 + t)*NB + b for head s, tensor t = 0 (query blocks) / 1 (key blocks), block b,
 *     NB = frames * blocks_per_frame; mean [..][64] fp32, split [..][128] fp16 bits, meta [..][2].
 *   idx: int32 [n][NB][frames*min(k, NBf)], frame-major, score descending, ties to the lower block.
 *   score(i, j) = sequential fmaf over d = 0..63 of mean_q[i][d] * mean_k[j][d], as saf3r_block_select.
 * Scores are approximated on the matrix cores from the split records with a proven error bound; a
 * (query block, frame) whose best k + 1 approximations are separated by more than the bound is
 * taken from them, every other one (near ties, rows flagged +inf) from the exact sequential scores
 * of its candidate keys, in the same kernel (one launch).
 *   workspace / workspace_bytes: not used (saf3r_block_select_pooled_workspace_bytes returns 0);
 *     NULL / 0 is accepted. They stay in the signature for callers built against ABI 12.
 * 1 <= k <= 32, blocks_per_frame <= 32 (k > 16 runs the sequential kernel on the means).
 * Replaces: the block top-k of the dynamic pattern (no reference symbol; per-frame semantics of
 *           saf3r/patch/wrapper.py:48 and saf3r/triton/fused_qk_topk.py:120-217 at block level).
 */
int saf3r_block_select_pooled(const float* mean, const uint16_t* split, const float* meta, int n, int frames,
                              int blocks_per_frame, int k, int32_t* idx, void* workspace, int64_t workspace_bytes,
                              void* stream);

/* Workspace bytes of saf3r_block_select_pooled for these sizes: 0 (the selection needs none), -1 for
 * sizes it rejects. No counterpart in the reference. */
int64_t saf3r_block_select_pooled_workspace_bytes(int n, int frames, int blocks_per_frame, int k);

/*
 * Mean query and probe scores of the q_probe_topk key set, for n_sel heads, from their fp32 q / k
 * rows (the saf3r_pack_qkv qk32 rows: row t of slot s at q32 + s*slot_stride + 64 t, k32 likewise).
 *   slots: device int32 [n_sel]; n_tokens: rows per slot (F*T); slot_stride >= 64 * n_tokens.
 *   sample_idx: device int32 [n_samples] token ids in [0, n_tokens) (entries outside are clamped),
 *               or NULL for every token (n_samples ignored). The reference's q_sample_ratio < 1
 *               samples torch.linspace(0, N-1, n).long() tokens; the caller passes that list.
 *   qbar[s][d]: mean over the sampled rows (all tokens without a list): chunks of ceil(M/256) rows
 *               (M rows in list order) summed sequentially, chunk sums added in order, one division
 *               by M.
 *   scores[s][t] (row stride scores_stride >= n_tokens, token order): sequential fmaf over d of
 *               qbar[d] * k[t][d], times scale (1/8 for head_dim 64).
 *   partial: device workspace of n_sel * 256 * 64 floats.
 * Replaces: saf3r/patch/sparse_attention.py:150-168 (query sampling, q_bar and the fp32 probe scores).
 */
int saf3r_probe_scores(const float* q32, const float* k32, int64_t slot_stride, int n_tokens, const int32_t* slots,
                       int n_sel, const int32_t* sample_idx, int n_samples, float scale, float* partial,
                       float* qbar, float* scores, int64_t scores_stride, void* stream);

/*
 * saf3r_probe_scores without the workspace argument: it allocates nothing (no hipMalloc / hipFree,
 * no allocating library call) and keeps the partial sums in a static device array of the library
 * (4 MiB per GPU, held until the process ends), for callers that cannot allocate: code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation. n_sel <= 64
 * (SAF3R_ERR_UNSUPPORTED beyond). Results are identical to saf3r_probe_scores. The array used is
 * the one of the device of `stream` (the current device for the NULL stream), shared by every call
 * on that device: calls that overlap on one GPU (other streams, other host threads) race. No
 * counterpart in the reference.
 */
int saf3r_probe_scores_noalloc(const float* q32, const float* k32, int64_t slot_stride, int n_tokens,
                               const int32_t* slots, int n_sel, const int32_t* sample_idx, int n_samples,
                               float scale, float* qbar, float* scores, int64_t scores_stride, void* stream);

/*
 * Shared key sets of n_heads heads (device int32 arrays of n_heads entries each):
 *   mode SAF3R_KEYSET_STRIDE: tokens t >= start with (t - start) % param == 0;
 *   mode SAF3R_KEYSET_TOPK:   the min(param, N) best scores[h][t] (row stride scores_stride),
 *                             ties to the lower token;
 *   include != 0: plus every token of frame 0 and every special token.
 *   idx[h] (row stride idx_stride >= N): the members in increasing token order; count[h]: their number.
 * Replaces: saf3r/patch/sparse_attention.py:170-178 (topk + unique) and :262-269 (strided + unique).
 */
int saf3r_keyset_build(const float* scores, int64_t scores_stride, int n_heads, const int32_t* mode,
                       const int32_t* param, const int32_t* start, const int32_t* include, int frames,
                       int tokens_per_frame, int num_special, int32_t* idx, int64_t idx_stride, int32_t* count,
                       void* stream);

/*
 * Compact K/V of the key sets, in the layout SAF3R_KEYSET heads read: for set s (head head_ids[s]),
 *   keyset_k: bf16 [n_sel][capacity][64], row j = packed K of token idx[s][j];
 *   keyset_v: bf16 [n_sel][capacity/64] transposed, permuted 64x64 tiles (as packed V) of the
 *             natural V rows v[t*v_tok_stride + h*v_head_stride + d].
 *   Tiles below ceil(count[s]/64) (at most max_tiles, max_tiles*64 <= capacity) are written,
 *   rows at or beyond count[s] as zeros.
 * Replaces: saf3r/patch/sparse_attention.py:181-182, :271-272 (k/v[:, :, idx, :]).
 */
int saf3r_keyset_gather(const void* k_packed, int frames, int tokens_per_frame, int num_special,
                        const int32_t* head_ids, int n_sel, const void* v, int64_t v_tok_stride,
                        int64_t v_head_stride, const int32_t* idx, int64_t idx_stride, const int32_t* count,
                        int max_tiles, void* keyset_k, void* keyset_v, int64_t capacity, void* stream);

/*
 * Block-sparse attention forward over the packed layout, every head in one launch.
 *   head_pattern: host int32 [num_heads] of saf3r_pattern ids.
 *   sel: int32 [n_block_dynamic][F*NBf][sel_width] block ids (-1 = empty), one list per
 *        BLOCK_DYNAMIC head in increasing head order; may be NULL when no head is BLOCK_DYNAMIC.
 *   out: bf16 natural layout, element (token t, head h, d) at out[t*out_row_stride + h*64 + d].
 *        TOKEN_DYNAMIC(_KEYSET) heads get only their special rows written here.
 *   scale: softmax scale (1/8 for head_dim 64).
 *   keyset_k / keyset_v / keyset_count / keyset_capacity: the saf3r_keyset_gather buffers of the
 *        KEYSET and TOKEN_DYNAMIC_KEYSET heads, set s serving the s-th of those heads in increasing
 *        head order; every query of a KEYSET head (every special row of a TOKEN_DYNAMIC_KEYSET head)
 *        attends keys 0 .. min(keyset_count[s], keyset_capacity)-1 (a count above the
 *        capacity is clamped to it; keyset_capacity is a multiple of 64). NULL / 0 when no head is KEYSET.
 *   bcast_q / bcast_k / bcast_v: frame 0 and per-frame buffers of the BROADCAST heads, b-th buffer
 *        for the b-th BROADCAST head in increasing head order, C = ceil(T/64)*64 rows per frame:
 *          bcast_q: bf16 [n_broadcast][C][64], row i = packed Q of token i (frame 0), zeros past T;
 *          bcast_k: bf16 [n_broadcast][C][64], the same for K;
 *          bcast_v: bf16 [n_broadcast][F][C/64] key-set V tiles (saf3r_keyset_gather layout) of
 *                   frame f's tokens f*T .. f*T+T-1.
 *        NULL when no head is BROADCAST.
 *   token_order: host uint8 [num_heads] or NULL: the saf3r_layout saf3r_pack_qkv packed each head
 *        in. SAF3R_LAYOUT_TOKEN is for DENSE heads (key and query tiles then cover the F*T tokens
 *        without padding), SAF3R_LAYOUT_FRAMED for FRAME_LOCAL / ANCHOR_LOCAL / ANCHOR heads (each
 *        query tile then walks whole frames: its own, frame 0, or both); any other pairing is an error.
 *   q_scaled: host uint8 [num_heads] or NULL: heads h < 64 whose Q rows (and BROADCAST Q buffer)
 *        hold q * scale * log2(e) rounded once to bf16 (saf3r_pack_qkv's q_scaled with that
 *        q_scale). Their walks take exp2 of the score MFMA results directly, without a running
 *        maximum; an item whose row sums do not end within [2^-64, 2^64] is walked again with
 *        the exact maximum. Same results within the bf16 tolerance.
 *   flags: 0 or SAF3R_ATTN_FIXED_ORDER. Without it, every key walk starts at the position the
 *        device's wall clock divided by the walk's step time points to, so that the work-groups
 *        resident at one moment read nearby key tiles (cache reuse); the summation order, and so the
 *        last bits of the output, then vary from run to run (always within the bf16 tolerance).
 *        The block lists of BLOCK_DYNAMIC heads are walked that way only when those heads' K and V
 *        rows exceed 256 MiB (the Infinity Cache); below, from their first position.
 *        With it, every walk starts at its first tile and the output is run-to-run identical.
 *   pace, pace_seq: the walks' step times. pace is NULL (default step times) or a caller-owned
 *        device array of 12 uint64, zero-filled once and passed to every call, with pace_seq
 *        counting the calls (0, 1, 2, ...): each call measures its walks' mean step time into the
 *        array and the next call starts its walks from that measurement. Calls on other streams that
 *        share one array only disturb the measurement, never results. Ignored with FIXED_ORDER.
 * Replaces: the per-head loop saf3r/patch/wrapper.py:94-106 and the mode implementations of
 *           saf3r/patch/sparse_attention.py:12-90 for full / global_to_frame / all_to_first / skip /
 *           stride / q_probe_topk (over their key sets) / broadcast_first, the dense special rows of
 *           dino_topk (:197-208), and the block-dynamic pattern.
 */
int saf3r_sparse_attn_fwd(const void* q_packed, const void* k_packed, const void* v_packed, int frames,
                          int tokens_per_frame, int num_special, int num_heads, const int32_t* head_pattern,
                          const int32_t* sel, int sel_width, float scale, void* out, int64_t out_row_stride,
                          const void* keyset_k, const void* keyset_v, const int32_t* keyset_count,
                          int64_t keyset_capacity, const void* bcast_q, const void* bcast_k,
                          const void* bcast_v, const uint8_t* token_order, const uint8_t* q_scaled, int flags,
                          unsigned long long* pace, unsigned int pace_seq, void* stream);

/*
 * Gather attention: out[r] = sum_j softmax_j(q[r] . k[idx[r][j]] * scale) v[idx[r][j]], fp32
 * scores and accumulation, head_dim 64 (q, k, v and out rows of 64 elements); idx entries < 0 or
 * >= num_keys are skipped; a row with no valid entry is written as zeros.
 *   q, k: bf16 rows, or fp32 rows with SAF3R_GATHER_QK_FP32 in dtype_flags;
 *   v: bf16 rows, or fp32 rows with SAF3R_GATHER_V_FP32; out: bf16 rows (the fp32 result rounded
 *   once), or fp32 rows with SAF3R_GATHER_OUT_FP32. Row strides are in elements of the row's type.
 *   (The reference upcasts q, k and v to fp32 and stores out in v.dtype: fp16 inputs are passed
 *   upcast to fp32 exactly, with an fp32 out rounded to fp16 by the caller.)
 *   idx: int32 [n][topk] (row stride topk, or 0 to share one list across rows).
 * Replaces: saf3r/triton/sparse_topk_attention.py:115-166 (fused_sparse_topk_attention) and
 *           :261-286 (the TopK > 2048 variant).
 */
int saf3r_gather_attn_fwd(const saf3r_rows* q, const saf3r_rows* k, const saf3r_rows* v, const int32_t* idx,
                          int64_t idx_row_stride, int n, int topk, int64_t num_keys, float scale, int dtype_flags,
                          const saf3r_rows* out, void* stream);
/*
 * saf3r_gather_attn_fwd in two passes, for many rows with long lists (the dino_topk image rows:
 * 128 frames x 1369 rows, 512 keys each): every row's list is cut into 8 slices of consecutive
 * entries; slice s is walked by work-groups the hardware places on XCD s (so each XCD's L2 holds
 * the rows of 1/8 of the list positions, one frame range for frame-major lists), each writing the
 * slice's partial softmax (maximum, sum of weights, unnormalised output) to the caller's workspace;
 * a second kernel merges the 8 partials of a row. Rows run in chunks of 65536 (both kernels per
 * chunk), so the workspace holds one chunk's partials. Same arguments and results as
 * saf3r_gather_attn_fwd within fp32 rounding (the summation order differs).
 *   workspace / workspace_bytes: caller-owned device memory of at least
 *     saf3r_gather_attn_workspace_bytes(n, topk) bytes, 16-byte aligned; calls that share it must
 *     be ordered (one stream).
 * Replaces: as saf3r_gather_attn_fwd.
 */
int saf3r_gather_attn_fwd_sliced(const saf3r_rows* q, const saf3r_rows* k, const saf3r_rows* v, const int32_t* idx,
                                 int64_t idx_row_stride, int n, int topk, int64_t num_keys, float scale,
                                 int dtype_flags, const saf3r_rows* out, void* workspace, int64_t workspace_bytes,
                                 void* stream);
/* Workspace bytes of saf3r_gather_attn_fwd_sliced (min(n, 65536) rows * 8 slices * 66 floats: at most
 * 138 MB), -1 for invalid sizes.
 * No counterpart in the reference (its kernel keeps each row's state in registers). */
int64_t saf3r_gather_attn_workspace_bytes(int n, int topk);

/*
 * Per-frame token top-k of q.k (bf16 inputs, fp32 MFMA accumulation), one batch element per call
 * (the reference's batch dimension B is a loop of calls over q[b], k[b], idx[b]).
 *   q: n_q rows; k: frames*per_frame rows (frame f = rows [f*per_frame, (f+1)*per_frame));
 *   idx: int32 [n_q][frames*min(topk, per_frame)] global key rows, frame-major, score descending,
 *   ties to the lower index. topk >= 1 and min(topk, per_frame) <= 128 (the reference's limit);
 *   above 16 per_frame <= 4096.
 *   workspace / workspace_bytes: caller-owned device memory for the scores of a chunk of queries,
 *   used when min(topk, per_frame) > 16 (NULL / 0 otherwise). saf3r_token_topk_workspace_bytes
 *   gives the size that runs every query in one chunk (at most about 1 GiB); any size of at least
 *   the scores of 128 queries (frames * roundup(per_frame, 64) * 4 * 128 bytes) works, in more
 *   chunks. Calls that share a workspace must be ordered (one stream).
 * Replaces: saf3r/triton/fused_qk_topk.py:120-217 (compute_qk_topk_indices_fused).
 */
int saf3r_token_topk(const saf3r_rows* q, const saf3r_rows* k, int n_q, int frames, int per_frame, int topk,
                     int32_t* idx, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes saf3r_token_topk takes for these sizes in one chunk: 0 when
 * min(topk, per_frame) <= 16, -1 for sizes saf3r_token_topk rejects. No counterpart in the
 * reference (its Triton kernel keeps each query's list in registers). */
int64_t saf3r_token_topk_workspace_bytes(int n_q, int frames, int per_frame, int topk);

/*
 * Token top-k from blocks of bf16 scores: the selection of the non-lazy DINO-feature path.
 *   scores: bf16 bits [rows][score_stride]; key j of frame f at column f*per_frame + j.
 *   per_frame_mode 1: the min(topk, per_frame) best keys of every frame (frames >= 1 with
 *     exclude_first), increasing key order within a frame, frame-major; 0: the min(topk, keys) best
 *     keys of the row (beyond frame 0 with exclude_first), in increasing key order.
 *   exclude_first: columns 0 .. ceil(per_frame/first_stride)-1 hold frame 0's samples 0, s, 2s, ...
 *     (s = first_stride > 0), the selected keys follow.
 *   cap > 0: at most cap selected keys (the best), in increasing key order; in per_frame_mode that
 *     needs cand_idx int32 / cand_key uint16 buffers of [rows][frames * min(topk, per_frame)].
 *   Ranking: the bf16 score, ties to the lower key. rows <= 65535, per_frame <= 4096.
 * Replaces: saf3r/patch/utils.py:54-184 (compute_qk_topk_indices_batched, its torch.topk selection,
 *           first-frame samples and max_topk cap).
 */
int saf3r_frame_topk_scores(const void* scores, int64_t score_stride, int rows, int frames, int per_frame,
                            int exclude_first, int first_stride, int per_frame_mode, int topk, int cap,
                            int32_t* idx, int64_t idx_stride, int32_t* cand_idx, uint16_t* cand_key, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAF3R_HIP_H */
