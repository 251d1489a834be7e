/*
 * fdl.h -- C ABI of the MI355X (gfx950) Flash-Cache hot path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream (passed as
 * `void*`, i.e. a hipStream_t; NULL means the null stream). Entry points validate their
 * scalar arguments on the host, enqueue kernels on the stream and return without
 * synchronising. Status: 0 on success, a negative FDL_ERR_* code otherwise; the text of
 * the last error of the calling thread is returned by fdl_last_error().
 *
 * Buffers are caller-owned. bf16 means IEEE bfloat16 stored as uint16. Row-major
 * everywhere. d_model = n_heads * head_dim; only head_dim == 128 is implemented.
 *
 * Table formats
 *   work item (int32 x 8), one per attention tile:
 *     [0] batch     row of the page table holding this sequence's pages
 *     [1] k_begin   first logical key position (inclusive)
 *     [2] k_end     last logical key position (exclusive), the reference's seqlen_k
 *     [3] row_off   offset into row_idx of this tile's query rows
 *     [4] n_rows    number of query rows (1..tile_rows, see fdl_block_attention)
 *     [5] n_imp     the first n_imp rows of the tile feed the importance scores
 *     [6] reserved  (0)
 *     [7] reserved  (0)
 *   page table (int32 [n_seq][max_pages]): logical key n of sequence b lives in cache
 *     slot page_table[b][n >> page_log2] * (1 << page_log2) + (n & ((1 << page_log2) - 1)).
 *     The reference's contiguous layout (slot = b*L + n) is the page table
 *     page_table[b][p] = b*L/P + p.
 *   verify block (int32 x 4): (k0, k1, q0, q1) exactly as the reference's verify block
 *     table: keys key_slots[k0..k1) from the cache, query rows [q0, q1) which are also
 *     the in-block keys.
 */
#ifndef FDL_H_
#define FDL_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FDL_ABI_VERSION 3

enum fdl_status {
  FDL_OK = 0,
  FDL_ERR_NULL = -1,        /* a required pointer is NULL */
  FDL_ERR_SHAPE = -2,       /* inconsistent or unsupported dimensions */
  FDL_ERR_RANGE = -3,       /* a table entry lies outside the buffer it indexes */
  FDL_ERR_UNSUPPORTED = -4, /* a valid request that the kernels do not implement */
  FDL_ERR_HIP = -5,         /* a HIP runtime call failed */
};

enum fdl_importance_mode {
  FDL_IMP_NONE = 0,
  /* sum over importance rows of the raw, unscaled logit q.k (flash_cache_triton.py:155-158) */
  FDL_IMP_RAW_LOGIT = 1,
  /* sum over importance rows of softmax(scale * q.k) probabilities (column sums) */
  FDL_IMP_SOFTMAX_COLSUM = 2,
};

/* Text of the calling thread's last error ("" if none). */
const char* fdl_last_error(void);

/* FDL_ABI_VERSION of the library. */
int fdl_abi_version(void);

/*
 * Fused QKV projection + rotate-half RoPE + K/V write.
 * Replaces the launches of _flash_qkv_proj_cache_fwd (flash_cache_triton.py:15-100,
 * launched at :541-559) and, with FDL_QKV_KV_PACKED, _flash_verify_qkv_proj_fwd
 * (flash_cache_triton.py:255-338, launched at :505-519).
 *
 *   x        bf16 [n_rows][d_model]         normalised hidden states (x_normed)
 *   wq/wk/wv bf16 [d_model][d_model]        nn.Linear weights, [out][in]
 *   rope_sin, rope_cos fp32 [n_rope_rows][head_dim]
 *   slot     int64 [n_rows]  cache slot of each row (the reference's query_pos_flat)
 *   rope_row int64 [n_rows]  row of the sin/cos tables for each row; NULL = use slot
 *   q_out    bf16 [n_rows][d_model]         rotated Q, packed by row
 *   k_out/v_out bf16: without FDL_QKV_KV_PACKED -> cache [n_kv_rows][d_model], row slot[r]
 *            is overwritten with the rotated K / V of row r; with it -> packed
 *            [n_rows][d_model] (n_kv_rows must equal n_rows).
 *   flags    FDL_QKV_KV_PACKED (1) and / or FDL_QKV_ROPE_HALVES_EQUAL (2): the caller
 *            asserts that every sin/cos row repeats its first half (rope_sin[r][c + head_dim/2]
 *            == rope_sin[r][c], the same for rope_cos), as the reference's tables do
 *            (cat(freqs, freqs), generate.py:44-50); only the first half of each row is read.
 * Rows whose slot or rope_row is out of range are skipped by the kernel; use
 * fdl_validate_rows to reject them on the host. x, the weights, the sin/cos tables and the
 * outputs must be 16-byte aligned (d_model is a multiple of 256).
 */
int fdl_qkv_rope_cache(const void* x, const void* wq, const void* wk, const void* wv,
                       const float* rope_sin, const float* rope_cos, int64_t n_rope_rows,
                       const int64_t* slot, const int64_t* rope_row, int64_t n_rows,
                       int64_t d_model, int64_t n_heads, int64_t head_dim, void* q_out,
                       void* k_out, void* v_out, int64_t n_kv_rows, int32_t flags,
                       void* stream);
enum { FDL_QKV_KV_PACKED = 1, FDL_QKV_ROPE_HALVES_EQUAL = 2 };

/*
 * Block-table attention over the KV cache for variable per-sequence query lengths, with
 * the importance side output.
 * Replaces _flash_masked_attention_fwd (flash_cache_triton.py:103-177, launched at
 * :561-577) and _flash_tracked_attention_fwd (:180-252, launched at :589-607) in one
 * launch: a tile may hold the masked rows and the tracked rows of one sequence, so the
 * sequence's K/V are streamed once. Bidirectional (no causal mask).
 *
 *   q        bf16 [n_q_rows][d_model]       rotated queries (q_out of fdl_qkv_rope_cache)
 *   k_cache, v_cache bf16 [n_slots][d_model]
 *   page_table int32 [n_seq][max_pages]; page size 1 << page_log2 (4 <= page_log2 <= 12)
 *   work     int32 [n_work][8] (see above); row_idx int32 [n_row_idx]
 *   tile_rows 64, 128 or 256: every work item of the call has at most tile_rows rows; 256
 *            selects the variant for full-recompute row sets, 128 and 64 the ones for mid and
 *            short ones. With tile_rows 256 and FDL_IMP_SOFTMAX_COLSUM the importance rows
 *            must lie in the first 128 rows of an item (n_imp <= 128).
 *   out      bf16 [n_q_rows][d_model]       rows named by row_idx are written
 *   imp_mode FDL_IMP_*; imp_part fp32 [n_heads][n_slots]: for every tile with n_imp > 0,
 *            imp_part[h][slot(n)] = sum over its first n_imp rows r of the head-h term
 *            (raw: q_r.k_n; softmax: exp(scale*q_r.k_n - lse_r)), for n in [k_begin, k_end).
 *            Slots of other tiles are left untouched. Reduce over heads with
 *            fdl_importance_accumulate. Each sequence must have at most one tile with
 *            n_imp > 0.
 *   workspace fp32 [workspace_floats], 16-byte aligned, or NULL / 0: with
 *            FDL_IMP_SOFTMAX_COLSUM, a 64-row tile with at most 32 importance rows
 *            and at most FDL_ATTN_ONCHIP_BLOCKS 64-key blocks keeps their probabilities on
 *            chip during its one pass over K/V; a longer one keeps them here: it needs
 *            FDL_ATTN_WS_FLOATS_PER_BLOCK floats per 64-key block for each head, and the room
 *            per tile is workspace_floats / (n_work * n_heads). A tile whose keys do not fit
 *            (or with more than 32 importance rows, or without a workspace) reads K a second
 *            time instead; the results are the same. Without softmax-colsum importance, a
 *            call of 64- or 128-row tiles whose n_work * n_heads workgroups fill at most a
 *            quarter of the device's compute units splits every tile's key blocks over
 *            p = min(FDL_ATTN_MAX_KV_PARTS, CUs / (n_work * n_heads)) workgroups when the
 *            workspace holds p * n_row_idx * n_heads * FDL_ATTN_PART_FLOATS floats (fewer
 *            parts when it holds less, none below 2, below 4 device-filling parts or without
 *            a workspace), and merges their partial rows in a second kernel: same attention
 *            within rounding, raw importance unchanged. Room for fewer than p parts but at
 *            least as many as the longest tile's 64-key blocks gives the same bits as room
 *            for p (part z of p takes blocks [z nb / p, (z + 1) nb / p): one block per
 *            non-empty part either way).
 *            Contents need no initialisation and are left undefined.
 */
#define FDL_ATTN_WS_FLOATS_PER_BLOCK (32 * 64 + 32)
#define FDL_ATTN_ONCHIP_BLOCKS 24
#define FDL_ATTN_PART_FLOATS 132
#define FDL_ATTN_MAX_KV_PARTS 8
int fdl_block_attention(const void* q, const void* k_cache, const void* v_cache,
                        int64_t n_q_rows, int64_t n_slots, int64_t d_model, int64_t n_heads,
                        int64_t head_dim, const int32_t* page_table, int64_t n_seq,
                        int64_t max_pages, int32_t page_log2, const int32_t* work,
                        int64_t n_work, const int32_t* row_idx, int64_t n_row_idx,
                        int32_t tile_rows, float softmax_scale, void* out, int32_t imp_mode,
                        float* imp_part, float* workspace, int64_t workspace_floats,
                        void* stream);

/*
 * No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops or harnesses that forbid hipMalloc): one call does
 * fdl_block_attention followed by fdl_importance_accumulate, with the per-head importance
 * partials (and, in what is left, fdl_block_attention's softmax-importance workspace) in a
 * library-owned static device array of FDL_NOALLOC_SCRATCH_BYTES (32 MiB) on each GPU, held
 * until the process ends, instead of caller workspaces. The caller still passes the inputs,
 * `out` and `scores`; nothing is allocated (no hipMalloc/hipFree).
 *   out     as fdl_block_attention
 *   scores  fp32 [n_slots], with imp_mode != FDL_IMP_NONE:
 *           scores[slot(n)] += imp_scale * sum_h (head-h importance of key n), heads summed in
 *           ascending order: bit for bit what fdl_block_attention + fdl_importance_accumulate
 *           (scale = imp_scale) leave in scores
 * Rejects (FDL_ERR_UNSUPPORTED) n_heads * n_slots * 4 bytes beyond FDL_NOALLOC_SCRATCH_BYTES.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (e.g. on two
 * streams) race on it and must be serialised by the caller.
 */
#define FDL_NOALLOC_SCRATCH_BYTES (32LL << 20)
int fdl_block_attention_scores_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                       int64_t n_q_rows, int64_t n_slots, int64_t d_model,
                                       int64_t n_heads, int64_t head_dim,
                                       const int32_t* page_table, int64_t n_seq,
                                       int64_t max_pages, int32_t page_log2, const int32_t* work,
                                       int64_t n_work, const int32_t* row_idx, int64_t n_row_idx,
                                       int32_t tile_rows, float softmax_scale, void* out,
                                       int32_t imp_mode, float imp_scale, float* scores,
                                       void* stream);

/*
 * scores[slot(n)] += scale * sum_{h = 0..n_heads-1} imp_part[h][slot(n)] for every tile
 * with n_imp > 0 and n in [k_begin, k_end), heads summed in ascending order.
 * Replaces `attn_scores += S.mean((0, 1)).view(-1)` (flash_cache_triton.py:614-615) with
 * scale = 1 / (block_m * n_heads).
 */
int fdl_importance_accumulate(const float* imp_part, int64_t n_heads, int64_t n_slots,
                              const int32_t* page_table, int64_t n_seq, int64_t max_pages,
                              int32_t page_log2, const int32_t* work, int64_t n_work,
                              float scale, float* scores, void* stream);

/*
 * Importance ranking of decoded slots (generate.py:364-366) and top-k gather (the
 * tracked refresh set, generate.py:375-381).
 *   scores fp32 [n_scores] indexed by slot
 *   slots  int64, segments seg[i] = (start, len) int32 [n_seg][2]: on return each segment
 *          slots[start .. start+len) is sorted ascending by (score, then slot descending),
 *          the reference's ascending sort with ties resolved so that among equal scores the
 *          lower slot ranks higher.
 *   topk_out int64 [n_seg][k] or NULL: the k highest-ranked slots of each segment, in rank
 *          order (score descending, slot ascending), -1 where a segment is shorter than k.
 *   max_len  upper bound of every len (<= 8192).
 */
int fdl_importance_rank(const float* scores, int64_t n_scores, int64_t* slots,
                        int64_t n_slot_entries, const int32_t* seg, int64_t n_seg,
                        int32_t max_len, int64_t* topk_out, int32_t k, void* stream);

/*
 * The step's last head reduction fused into the ranking. Segment i belongs to the sequence
 * in page-table row seg_keys[i][0], whose keys are n in [0, seg_keys[i][1]); for each of
 * those keys (slot = slot(row, n) in [0, n_scores))
 *   scores[slot] = fma(scale, sum_{h = 0..n_heads-1} imp_part[h][slot], scores[slot])
 * (heads summed in ascending order: bit for bit what fdl_importance_accumulate stores for
 * a tile of that sequence with keys [0, k_end)), then the segment is ranked and its top-k
 * gathered as by fdl_importance_rank. Replaces, at a step's last layer,
 * `attn_scores += S.mean((0, 1))` (flash_cache_triton.py:614-615) followed by the sort of
 * generate.py:364-366 and the gather of :375-381. Segment entries that are not keys of
 * their sequence keep their score. A page-table row may appear in at most one segment.
 *   imp_part fp32 [n_heads][n_scores] (fdl_block_attention's per-head importance)
 *   seg_keys int32 [n_seg][2]
 */
int fdl_importance_accumulate_rank(const float* imp_part, int64_t n_heads, float scale,
                                   const int32_t* page_table, int64_t n_seq, int64_t max_pages,
                                   int32_t page_log2, const int32_t* seg_keys, float* scores,
                                   int64_t n_scores, int64_t* slots, int64_t n_slot_entries,
                                   const int32_t* seg, int64_t n_seg, int32_t max_len,
                                   int64_t* topk_out, int32_t k, void* stream);

/*
 * Flash-Verify attention. Replaces _flash_verify_attention_fwd (flash_cache_triton.py:
 * 341-428, launched at :523-535): for each verify block (k0, k1, q0, q1) and head, the
 * rows [q0, q1) attend to the cache keys key_slots[k0..k1) and to the block's own rows
 * as in-block keys (k_blk/v_blk, packed by row) under the block's boolean mask.
 *   q, k_blk, v_blk bf16 [n_q_rows][d_model]    (outputs of fdl_qkv_rope_cache, FDL_QKV_KV_PACKED)
 *   key_slots int64 [n_keys]
 *   vblocks  int32 [n_vblocks][4]; q1 - q0 <= block_rows <= 256 (the reference's 2 * block_m)
 *   exactly one of
 *   mask     uint8 [n_vblocks * block_rows][block_rows]; row i of block v is
 *            mask[v*block_rows + i]; nonzero = may attend (the reference's attn_mask), or
 *   vmeta    int32 [n_vblocks][2] = (T, S): the block's rows are T fill rows, S draft rows
 *            and S mask rows (T + 2S = q1 - q0), and the mask is the reference's closed form
 *            (generate.py:260-269): fill rows do not see the drafts, draft i sees drafts
 *            j <= i and masks j > i, mask i sees drafts j < i and masks j >= i, all else is
 *            visible. No mask is read from memory.
 *   Column j is additionally valid only if q0 + j < q1.
 *   out      bf16 [n_q_rows][d_model]
 * Softmax is exact over the union of both key sets (the running maximum includes the
 * in-block logits).
 */
int fdl_verify_attention(const void* q, const void* k_blk, const void* v_blk,
                         const void* k_cache, const void* v_cache, int64_t n_q_rows,
                         int64_t n_slots, int64_t d_model, int64_t n_heads, int64_t head_dim,
                         const int64_t* key_slots, int64_t n_keys, const int32_t* vblocks,
                         int64_t n_vblocks, const uint8_t* mask, const int32_t* vmeta,
                         int32_t block_rows, float softmax_scale, void* out, void* stream);

/*
 * Host-side validators (host pointers; no GPU needed). They return FDL_ERR_RANGE with a
 * message naming the first offending entry.
 */
/*
 * Fused elementwise parts of the block around the hot path (one HBM pass each).
 *
 * fdl_rms_norm replaces `x_normed = self.attn_norm(x)` (flash_cache_triton.py:494, the
 * RMSLayerNorm of modeling_llada.py:389-403) and, with a residual, the sequence
 * `x = x + att; og_x = x; x = self.ff_norm(x)` (flash_cache_triton.py:618-624):
 *   s = bf16(x + residual) -> sum_out (residual may be NULL: s = x, sum_out unused)
 *   out = bf16(weight * bf16(s * rsqrt(mean(s^2) + eps)))
 *   x, residual, sum_out, out bf16 [n_rows][d]; weight bf16 [d]; d % 8 == 0, d <= 8192.
 */
int fdl_rms_norm(const void* x, const void* residual, const void* weight, int64_t n_rows,
                 int64_t d, float eps, void* sum_out, void* out, void* stream);

/*
 * fdl_silu_mul replaces `x = self.act(x); x = x * x_up` with the SiLU activation
 * (flash_cache_triton.py:628-633): out = bf16(bf16(silu(gate)) * up), n elements (n % 8 == 0).
 */
int fdl_silu_mul(const void* gate, const void* up, int64_t n, void* out, void* stream);

/*
 * fdl_silu_mul_rows: the same over n_rows rows whose gate and up halves are strided views,
 * e.g. the two halves of one [n_rows][2 * width] product of the concatenated ff_proj / up_proj
 * weights (one GEMM instead of the two at flash_cache_triton.py:628):
 *   y[r][c] = bf16(bf16(silu(gate[r * ld + c])) * up[r * ld + c]).
 * The output is cut into out_chunks column chunks of w = width / out_chunks columns, stored
 * chunk after chunk: y[r][c] at out[(c / w) * n_rows * w + r * w + c % w] ([out_chunks][n_rows][w];
 * out_chunks = 1 is plain [n_rows][width] rows). The chunked form is the K-split operand of
 * a split-K ff_out product. width and ld multiples of 8, ld >= width, w a multiple of 8; all
 * pointers 16-byte aligned.
 */
int fdl_silu_mul_rows(const void* gate, const void* up, int64_t n_rows, int64_t width,
                      int64_t ld, int64_t out_chunks, void* out, void* stream);

/*
 * fdl_split_reduce_residual: the end of a split-K ff_out product with its residual
 * (flash_cache_triton.py:634-636, `x = og_x + ff_out(x)`):
 *   residual_out[i] = bf16(float(residual_out[i]) + (part[0][i] + part[1][i] + ...)),
 * one rounding, as a GEMM that accumulates into the residual (beta = 1) rounds once.
 *   part fp32 [n_split][n_rows][n_cols]; residual_out bf16 [n_rows][n_cols], updated in place;
 *   n_cols % 8 == 0, pointers 16-byte aligned.
 */
int fdl_split_reduce_residual(const float* part, int64_t n_split, int64_t n_rows,
                              int64_t n_cols, void* residual_out, void* stream);

/*
 * LM-head confidence. Replaces, for bf16 logits rows [n_rows][vocab] (contiguous, 16-byte
 * aligned, vocab a multiple of 8):
 *   token == NULL: p = softmax(logits.to(float64), -1); prob, arg = max(p, -1)
 *                  (generate.py:218, :320): prob[r] = the float64 softmax maximum of row r,
 *                  arg[r] (if arg != NULL) = the first index of the row's maximum logit;
 *   token != NULL: prob[r] = softmax(logits[r].to(float64))[token[r]] (generate.py:337),
 *                  0 for a token outside [0, vocab); arg[r] as above if arg != NULL.
 * The float64 terms are the same as torch's; the order of the float64 sum differs.
 */
int fdl_softmax_confidence(const void* logits, int64_t n_rows, int64_t vocab,
                           const int64_t* token, double* prob, int64_t* arg, void* stream);

/*
 * Device-side decode scheduler (the bookkeeping of generate.py:125-470 in device memory; one
 * host synchronisation per denoising step). Every pointer is device memory; the struct is
 * read on the host at each call (pass it by host pointer).
 *
 * Per-sequence state seq int32 [n_seq][FDL_SCHED_SEQ_FIELDS] (field indices below); token
 * ids x / x_draft int64 [n_seq * max_length] and the slot order full_pos int64
 * [n_seq][max_length] hold logical slots j * max_length + p, as the reference's tensors do.
 * A row with seq[ACTIVE] < 0 is idle. A newly admitted row has FRESH = 1, ND = its prompt
 * length, EOS = -1, PRED = the reference's predicted_length, SEQLEN_K its key count.
 */
enum fdl_sched_seq_field {
  FDL_SEQ_ACTIVE = 0,     /* prompt index, -1: idle row */
  FDL_SEQ_ND = 1,         /* decoded count (num_decoded) */
  FDL_SEQ_SEQLEN_K = 2,   /* keys of the sequence (seqlen_k) */
  FDL_SEQ_PRED = 3,       /* predicted_length (a slot bound) */
  FDL_SEQ_EOS = 4,        /* decoded_eos_pos (a slot) or -1 */
  FDL_SEQ_N_MASKED = 5,   /* masked rows of the step: full_pos[ND : ND + N_MASKED] */
  FDL_SEQ_KEEP = 6,       /* tokens accepted by the step's last acceptance stage */
  FDL_SEQ_T = 7,          /* verify fill rows */
  FDL_SEQ_S = 8,          /* verify candidates */
  FDL_SEQ_DONE = 9,       /* 1: nothing left before the predicted length */
  FDL_SEQ_N_TRACKED = 10, /* tracked rows: full_pos[T0 : ND] then full_pos[ND + block_m : T1] */
  FDL_SEQ_T0 = 11,
  FDL_SEQ_T1 = 12,
  FDL_SEQ_FRESH = 13,     /* 1: the next step recomputes every slot (step 0 of a prompt) */
  FDL_SEQ_ERR = 14,       /* 1: fewer decoded slots than verify fill rows */
  FDL_SEQ_HI = 15,        /* highest position (p of slot j * L + p) the next step's rows
                             query, -1: none (a paged pool grows the row's pages to it) */
  FDL_SCHED_SEQ_FIELDS = 16,
};
/* summary int32 [FDL_SCHED_SUMMARY_FIELDS], written by fdl_sched_pack (DECODED and
 * VERIFY_ACCEPTED are running totals the caller may reset) */
enum fdl_sched_summary_field {
  FDL_SUM_Q = 0,              /* packed rows of the next forward */
  FDL_SUM_N_MASKED_ROWS = 1,  /* its first rows, the masked ones (the LM head rows) */
  FDL_SUM_N_LONG = 2,         /* work items: long (256-row) tiles, then mid, then short */
  FDL_SUM_N_MID = 3,
  FDL_SUM_N_SHORT = 4,
  FDL_SUM_N_CONT = 5,         /* active rows that continue */
  FDL_SUM_N_DONE = 6,         /* active rows that finished (DONE = 1) */
  FDL_SUM_OVERFLOW = 7,       /* 1: rows or items beyond q_cap / work_cap (nothing written) */
  FDL_SUM_DECODED = 8,
  FDL_SUM_VERIFY_ACCEPTED = 9,
  FDL_SCHED_SUMMARY_FIELDS = 16,
};
typedef struct fdl_sched {
  int64_t* x;          /* token ids */
  int64_t* x_draft;    /* pass-1 draft tokens */
  int64_t* full_pos;   /* slot order */
  int32_t* seq;        /* per-sequence fields */
  int32_t* summary;
  /* next forward (fdl_sched_pack): packed slots and token ids, work items of
   * fdl_block_attention (long, mid, short tiles in that order) and their row lists */
  int64_t* qpos;       /* [q_cap] */
  int64_t* xq;         /* [q_cap] */
  int32_t* row_idx;    /* [q_cap] */
  int32_t* work;       /* [work_cap][8] */
  /* ranking segments (start, len) of the active rows, in row order (acceptance kernels) */
  int32_t* seg;        /* [n_seq][2] */
  /* Flash-Verify lists of the active rows (fdl_sched_pass1 with verify = 1): block a holds
   * packed rows [2 block_m a, 2 block_m (a + 1)) */
  int64_t* vpos;       /* [n_seq * 2 block_m] slots of the verify rows */
  int64_t* xv;         /* [n_seq * 2 block_m] their token ids */
  int64_t* key_pos;    /* [n_seq * max_length] cache keys of the blocks, packed */
  int32_t* vblocks;    /* [n_seq][4] (k0, k1, q0, q1) */
  int32_t* vmeta;      /* [n_seq][2] (T, S) */
  int64_t* draft_tok;  /* [n_seq * block_m / 2] draft token of the last block_m / 2 rows of
                          each block (its mask rows are the last S of them), -1 elsewhere */
  int64_t n_seq, max_length, q_cap, work_cap;
  int32_t block_m, track_num, mask_num, verify;
  int64_t eos_id;
  double threshold, gamma;
} fdl_sched;

/* Pass-1 acceptance from the masked rows' float64 confidences and tokens
 * (fdl_softmax_confidence over the first FDL_SUM_N_MASKED_ROWS rows) and, with verify, the
 * verify lists. Replaces generate.py:215-258 (with Flash-Verify), :335-350 (without) and
 * :260-297. */
int fdl_sched_pass1(const fdl_sched* state, const double* conf, const int64_t* tok,
                    void* stream);
/* Verify acceptance from the float64 probability of each block's draft tokens on its last
 * block_m / 2 rows (fdl_softmax_confidence with draft_tok). Replaces generate.py:307-333. */
int fdl_sched_verify_accept(const fdl_sched* state, const double* prob, void* stream);
/* Completion test and the next step's masked / tracked rows, packed, with the attention
 * work items; the summary. Replaces generate.py:364-383 (after the ranking) and :439-467. */
int fdl_sched_pack(const fdl_sched* state, void* stream);

/*
 * Attention work list from the reference's block tables, on the device: no host copy of
 * the tables. The reference's attention launches consume its masked and tracked block
 * tables (rows (batch, k_end, q0, q1), generate.py:52-58, :146-163, :439-465; launched at
 * flash_cache_triton.py:561-607); this builds the work items and row list that
 * fdl_block_attention takes from them.
 *   masked, tracked int64 [n][4] (device), any number of entries (n_masked + n_tracked
 *   < 2^30; the tables pass through the workgroup's LDS in chunks of 1024 entries)
 *   rows of a (batch, k_end) pair are grouped in order of first appearance: its masked rows
 *   (the importance rows) then its tracked rows; at most 1024 such pairs (the reference
 *   has one k_end per batch row). A group of up to 64 rows is one 64-row tile, up to 128 one
 *   128-row tile, more one 256-row tile per 256 rows. n_seq <= 1024.
 *   work int32 [cap_long + cap_mid + cap_short][8], 16-byte aligned: the 256-row tiles from
 *   item 0, the 128-row tiles from item cap_long, the 64-row tiles from cap_long + cap_mid;
 *   unused items are zero (no rows, no keys), which fdl_block_attention and
 *   fdl_importance_accumulate skip, so each region can be launched whole. cap_long =
 *   n_q_rows / 128 and cap_mid = cap_short = n_seq always suffice.
 *   row_idx int32 [n_q_rows]; status int32 [4] (16-byte aligned) or NULL: tiles of each
 *   class and error flags (1: an entry out of range, dropped; 2: more rows than n_q_rows,
 *   the groups past n_q_rows get no tiles; 4: a region over capacity; 8: more than 256
 *   importance rows in a group; 16: more than 1024 (batch, k_end) groups, the entries of
 *   the further groups dropped).
 * One workgroup; enqueued on `stream`.
 */
int fdl_work_from_blocks(const int64_t* masked, int64_t n_masked, const int64_t* tracked,
                         int64_t n_tracked, int64_t n_seq, int64_t n_q_rows, int64_t max_k,
                         int32_t* work, int64_t cap_long, int64_t cap_mid, int64_t cap_short,
                         int32_t* row_idx, int32_t* status, void* stream);

/* every slot in [0, n_kv_rows), every rope_row (or slot when rope_row is NULL) in
 * [0, n_rope_rows), and no slot repeated (two rows writing one cache row race). */
int fdl_validate_rows(const int64_t* slot, const int64_t* rope_row, int64_t n_rows,
                      int64_t n_kv_rows, int64_t n_rope_rows, int32_t kv_packed);
/* work items, their row lists and page-table entries lie inside their buffers. */
int fdl_validate_work(const int32_t* work, int64_t n_work, const int32_t* row_idx,
                      int64_t n_row_idx, int64_t n_q_rows, const int32_t* page_table,
                      int64_t n_seq, int64_t max_pages, int32_t page_log2, int64_t n_slots);
/* verify blocks and their key lists lie inside their buffers. */
int fdl_validate_vblocks(const int32_t* vblocks, int64_t n_vblocks, const int64_t* key_slots,
                         int64_t n_keys, int64_t n_q_rows, int64_t n_slots,
                         int32_t block_rows);

#ifdef __cplusplus
}
#endif

#endif /* FDL_H_ */
