/*
 * ds355 — MI355X (gfx950) DiffSpec draft-context retrieval: C ABI.
 *
 * One shared library, libds355.so, built from hand-written HIP kernels.
 * Every entry point:
 *   - takes plain device pointers, element strides and sizes (no torch types);
 *   - launches asynchronously on the caller's HIP stream and never
 *     synchronises the host, never reads device values back and never
 *     allocates device memory (all buffers are owned by the caller);
 *   - returns 0 on success or a DS_ERR_* code; ds_last_error() then holds a
 *     message (thread-local, valid until the next call on that thread).
 * Strides are in elements, not bytes.  Reference citations are relative to
 * the vllm-ascend-hust-diffspec repository root.
 */
#ifndef DS355_H
#define DS355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ds_stream_t; /* == hipStream_t */

enum ds_dtype { DS_BF16 = 0, DS_FP16 = 1, DS_FP32 = 2 };

enum ds_status {
  DS_OK = 0,
  DS_ERR_INVALID = 1,     /* argument / shape check failed            */
  DS_ERR_UNSUPPORTED = 2, /* valid but outside what the kernels cover */
  DS_ERR_HIP = 3          /* a HIP runtime call failed                */
};

enum ds_head_reduce { DS_HEAD_MEAN = 0, DS_HEAD_MAX = 1 };

/* Message for the last failed call on this thread ("" after success). */
const char* ds_last_error(void);

/* ABI version, bumped on any signature change. */
int ds_abi_version(void);

/*
 * Paged chunk scores.
 * Replaces paged_chunk_attention_scores (diffspec/kernels.py:95-150) and its
 * Triton kernel (diffspec/kernels.py:11-92).
 *
 *   out[b, c] = reduce_h( sum_{t in chunk c, t < seq_lens[b]}
 *                           exp(scale * q[b,h] . k[t, h / (Hq/Hkv)] - lse[b,h]) )
 *               / max(n_valid(b, c), 1)
 * with reduce_h = mean over the Hq query heads (the reference) or max over
 * heads per token (DS_HEAD_MAX).  Keys are read through
 * block_table[b * bt_stride + t / block_size].  out is [batch, max_chunks]
 * fp32 with row stride out_stride; chunks at or beyond ceil(seq_lens[b] /
 * chunk) are written as 0, as the reference does.
 *
 * query   : [batch, Hq, head_dim], token stride q_stride, head stride head_dim.
 * lse     : fp32, element (b, h) at lse[b * lse_row_stride + h * lse_head_stride];
 *           NULL computes it: each query head's logsumexp over the row's
 *           scored tokens, in the same pass over the keys (the reference's
 *           chunk_attention_scores with softmax_lse=None,
 *           diffspec/runtime.py:321-322); head mean only.
 * key_cache: element (block, i, kvh, d) at
 *            k[block * k_block_stride + i * k_token_stride + kvh * k_head_stride + d].
 * dtype   : DS_BF16 or DS_FP16 (query and key_cache share it).
 * workspace: caller-owned device scratch of batch * max_chunks * Hkv floats
 *           (per-KV-head partial sums; unused with DS_HEAD_MAX), plus,
 *           when lse is NULL, batch * max_chunks * Hq * 2 floats of
 *           mass words (one 64-bit word per chunk and query head: the
 *           chunk's log2 mass as fp32 in its low half) and batch * Hq
 *           floats of row LSEs (placed first; the workspace must be 8-byte
 *           aligned).  Two
 *           kernels (four without an LSE): the streaming pass, the head
 *           LSEs, the partials and a small finalize pass.
 * Limits  : head_dim % 32 == 0 and <= 256, Hq % Hkv == 0, Hq / Hkv <= 16,
 *           batch <= 1024; DS_HEAD_MAX needs chunk <= 128 or a chunk that
 *           divides 64.
 */
int ds_chunk_scores(ds_stream_t stream, int dtype,
                    const void* query, int64_t q_stride,
                    const void* key_cache, int64_t k_block_stride,
                    int64_t k_token_stride, int64_t k_head_stride,
                    const float* lse, int64_t lse_row_stride, int64_t lse_head_stride,
                    const int32_t* block_table, int64_t bt_stride,
                    const int32_t* seq_lens,
                    int batch, int num_q_heads, int num_kv_heads, int head_dim,
                    int block_size, int chunk_size, int max_chunks, float scale,
                    int head_reduce, float* out, int64_t out_stride,
                    float* workspace, size_t workspace_bytes);

/*
 * Batched top-k chunk selection.
 * Replaces select_context_chunks (diffspec/runtime.py:348-414), called per
 * row from runtime.py:1298-1308, as one launch over all rows.
 *
 * For row b with C = ceil(seq_lens[b] / chunk) and K = history_budget / chunk:
 * C <= K selects 0..C-1; otherwise the newest chunk C-1 plus the K-1 highest
 * scores of chunks 0..C-2 (equal scores: the lower chunk index wins), all in
 * ascending order.  Writes ids[b * ids_stride + j] for j < counts[b] and
 * counts[b].  ids_stride >= K.  seq_lens[b] is clamped to score_cols * chunk
 * (the columns the score buffer holds).  Limits: K <= 2048, batch <= 65535.
 */
int ds_select_chunks(ds_stream_t stream,
                     const float* scores, int64_t score_stride, int score_cols,
                     const int32_t* seq_lens, int batch,
                     int chunk_size, int history_budget,
                     int32_t* ids, int64_t ids_stride, int32_t* counts);

/*
 * History plans from per-slot selections.
 * Replaces _history_plan_host + the plan tensor build
 * (diffspec/runtime.py:1713-1757) without host round trips.
 *
 * Row r uses slot = slots[r] and history_end = max(0, committed_lens[r] - 1).
 * sel_count[slot] < 0 means "no selection" (window of the last
 * history_budget tokens), 0 an empty selection, > 0 the number of sorted
 * chunk ids at sel_ids[slot * sel_stride].  The rolling tail is
 * min(history_end, recent_window, history_budget) tokens (recent_window ==
 * chunk_size is the reference).  plan is [rows, plan_width] int64:
 * [slot, history_len, tail_start, prefix_len, prefix_drop, chunk_ids..., 0...]
 * (diffspec/compact_kv.py:197-205); plan_width = 5 + token_budget / chunk.
 * working_lens[slot] = history_len when working_lens is not NULL.
 * Rows with slots[r] outside [0, num_slots) are padding: plan row of zeros,
 * no other write.
 */
int ds_build_plan(ds_stream_t stream,
                  const int32_t* sel_ids, int64_t sel_stride, const int32_t* sel_count,
                  int num_slots, const int32_t* slots, const int32_t* committed_lens, int rows,
                  int chunk_size, int history_budget, int recent_window,
                  int64_t* plan, int plan_width, int32_t* working_lens);

/*
 * Gather + local-position RoPE + working-cache write from plans.
 * Replaces rebuild_compact_kv_from_plan (diffspec/compact_kv.py:184-242) and
 * its Triton kernel (diffspec/compact_kv.py:8-133).
 *
 * raw  : [num_slots, max_model_len, heads, head_dim] (contiguous).
 * work : [num_slots, heads, token_budget, head_dim] (contiguous).
 * plan : [rows, plan_width] int64 (format above), contiguous.
 * cos_sin: [cs_rows, >= rotary_dim], row stride cs_stride; cos at [p, i],
 *          sin at [p, rotary_dim/2 + i].
 * For each row and local position p < min(history_len, roundup16(max_width)):
 * K[:rotary_dim] rotated at position p in fp32 (neox halves or GPT-J pairs),
 * K[rotary_dim:] and V copied.  Nothing else is written.  row_active, if not
 * NULL, skips rows with row_active[r] == 0.  dtype: DS_BF16/FP16/FP32.
 */
int ds_rebuild_compact_kv(ds_stream_t stream, int dtype,
                          const void* raw_key, const void* raw_value,
                          void* working_key, void* working_value,
                          const int64_t* plan, int rows, int plan_width,
                          const void* cos_sin, int64_t cs_stride, int cs_rows,
                          int num_slots, int max_model_len, int heads, int head_dim,
                          int token_budget, int chunk_size, int rotary_dim,
                          int is_neox_style, int max_width, const int32_t* row_active);

/*
 * One fused retrieval step (no reference counterpart as a single call; it is
 * runtime.py:1211-1308 + 1737-1765 + compact_kv.py as one launch chain):
 *   DS_STAGE_SCORE : score rows with counts > 0 (committed query, rejected
 *                    suffix cut; rows >= batch_size are padding)
 *   DS_STAGE_SELECT: select into the per-slot state (rows with counts > 0)
 *   DS_STAGE_PLAN  : plan row for every row from the slot state, then
 *                    gather / RoPE / write
 * `stages` is a bit mask; all three = one retrieval step.  SELECT and PLAN
 * share one kernel launch.  At most three kernels on `stream`, no host
 * synchronisation, launch shapes fixed by the descriptor's upper bounds
 * (graph-capturable).  With all three stages and a workspace, shapes the
 * fused kernel covers (bf16/fp16 KV, head_dim 64 or 128, <= 8 KV heads,
 * 8 to 256 batch rows, 16-token-aligned pages) run as one launch with the
 * same results, with a supplied LSE or without one.
 */
enum ds_stage { DS_STAGE_SCORE = 1, DS_STAGE_SELECT = 2, DS_STAGE_PLAN = 4, DS_STAGE_ALL = 7, DS_STAGE_PREFIX = 8 };

/*
 * DS_STAGE_PREFIX (in place of DS_STAGE_PLAN): plan rows and working_lens as
 * DS_STAGE_PLAN writes them, but only the gather tasks whose raw rows all lie
 * below the first row the draft's prefill of this step rewrites (each row's
 * first verifier query position, target_len - query_len) are moved: the
 * history prefix and the rolling tail up to that row.  The retrieval call can
 * move them before populate_prefill; the compact prefill then finds them
 * recorded and moves only the rest (the verifier's accepted positions).
 * Needs gather records (below) and DS_STAGE_SELECT in the same call (it reads
 * the verifier rows); committed_lens may be NULL (each row's scored length is
 * used, 0 for rows that committed nothing).  SCORE | SELECT | PREFIX with a
 * workspace runs as the single launch.
 *
 * Gather records (sel_gen and gather_rec, both or neither): per slot, the
 * selection generation, which every stored selection increments (the caller
 * increments it too when a different request takes the slot), and per
 * (slot, gather task of the plan's local positions) what the working cache
 * holds: (generation << 32) | (prefix drop + 1) for a task wholly inside the
 * history prefix, (generation << 32) | 2^31 | history end (the root
 * position) for another task wholly inside the history, else 0.  A PLAN or
 * PREFIX gather leaves out every task whose record already matches the plan,
 * since its bytes would not change, and keeps the records.  Raw rows before a
 * request's committed root must not change while the request holds its slot,
 * and the working cache only at and past each history's end.  Zero-filled by
 * the owner.
 */

typedef struct ds_step_desc {
  /* verifier snapshot (scoring) */
  int dtype;                         /* DS_BF16 / DS_FP16                     */
  const void* query;                 /* [num_query_tokens, Hq, D]             */
  int64_t q_stride;                  /* elements between query tokens         */
  const float* lse;                  /* (token, h) at lse[t*lse_token_stride + h*lse_head_stride] */
  int64_t lse_token_stride, lse_head_stride;
  const void* key_cache;             /* paged target keys                     */
  int64_t k_block_stride, k_token_stride, k_head_stride;
  int block_size;
  const int32_t* block_table;        /* [batch_rows, *] row stride bt_stride  */
  int64_t bt_stride;
  const int32_t* counts;             /* [batch_rows] committed tokens (0 = none) */
  const int32_t* query_start;        /* [batch_rows] first query token of row */
  const int32_t* query_len;          /* [batch_rows] query tokens of row      */
  const int32_t* target_len;         /* [batch_rows] verifier KV length       */
  int batch_rows;                    /* rows in the (padded) batch            */
  int batch_size;                    /* real rows; rows >= batch_size are padding */
  int num_q_heads, num_kv_heads, head_dim;
  float scale;
  int max_chunks;                    /* >= ceil(max scored length / chunk)    */
  float* scores;                     /* [batch_rows, max_chunks] final scores (written by SELECT) */
  float* score_partials;             /* [batch_rows, max_chunks, Hkv] per-KV-head sums (SCORE -> SELECT) */
  int stages;                        /* DS_STAGE_* bit mask                   */
  /* selection state, per slot */
  int32_t* sel_ids;                  /* [num_slots, sel_stride]               */
  int64_t sel_stride;                /* >= token_budget / chunk               */
  int32_t* sel_count;                /* [num_slots]  -1 none / 0 empty / n    */
  const int32_t* slots;              /* [batch_rows] canonical slot per row, -1 padding */
  /* plan */
  const int32_t* committed_lens;     /* [batch_rows] root position + 1        */
  int64_t* plan;                     /* [batch_rows, plan_width]              */
  int plan_width;
  int32_t* working_lens;             /* [num_slots] or NULL                   */
  /* draft raw / working caches */
  int kv_dtype;                      /* DS_BF16 / DS_FP16 / DS_FP32           */
  const void* raw_key; const void* raw_value;
  void* working_key; void* working_value;
  int num_slots, max_model_len, draft_heads, draft_head_dim, token_budget;
  const void* cos_sin; int64_t cs_stride; int cs_rows;
  int rotary_dim, is_neox_style;
  const int32_t* row_active;         /* [batch_rows] or NULL: rows to re-gather */
  /* policy */
  int chunk_size, history_budget, recent_window;
  /* single-launch step: zero-filled once, ds_step_workspace_bytes() bytes,
   * 64-byte aligned; NULL runs the kernel chain */
  void* workspace;
  size_t workspace_bytes;
  /* scoring without a supplied LSE (lse == NULL): the pass computes each
   * query head's LSE over the row's scored tokens (the reference's
   * chunk_attention_scores with softmax_lse=None, diffspec/runtime.py:321-322).
   * lse_partials holds one 64-bit word per (row, chunk, query head), 8-byte
   * aligned; the single launch tags its words with the workspace's launch
   * tags, so one lse_partials buffer serves one workspace (or is zeroed when
   * it moves to another) */
  float* lse_partials;               /* [batch_rows, max_chunks, Hq, 2] fp32 scratch; required when lse == NULL */
  float* lse_out;                    /* [batch_rows, Hq] natural-log LSE of each scored row; required when lse == NULL */
  int64_t lse_out_stride;            /* elements between rows of lse_out */
  int flags;                         /* DS_STEP_* bits; 0 for normal use */
  /* gather records (see DS_STAGE_PREFIX), or both NULL */
  int32_t* sel_gen;                  /* [num_slots] selection generations     */
  uint64_t* gather_rec;              /* [num_slots, rec_stride], rec_stride >= token_budget */
  int64_t rec_stride;
} ds_step_desc;

/*
 * ds_step_desc.flags, for tests of the single launch's rare paths; 0 in
 * normal use.
 *   DS_STEP_SELECTORS_GATHER: the scoring waves leave every gather task to
 *     the last workgroup to finish, the path a task takes when its scoring
 *     wave gave up waiting for the plan.  Same results, slower.
 *   DS_STEP_EXPIRE_WAITS: every selector reports an expired wait (status
 *     bit 0), so the launch's bounded waits stop early and its results are
 *     not valid; every wave still finishes.  Tests that one launch's expiry
 *     is handed to the owner's status word and does not reach the next.
 */
enum ds_step_flags { DS_STEP_SELECTORS_GATHER = 1, DS_STEP_EXPIRE_WAITS = 2 };

int ds_retrieval_step(ds_stream_t stream, const ds_step_desc* desc);

/*
 * Workspace of the single-launch step for these buffer sizes (0 when one of
 * them is not positive).  No reference counterpart: it holds the stages'
 * hand-over state (64 header bytes; a tagged copy of each plan row, 128
 * 8-byte columns per row; a 4-byte skip mark per gather task,
 * ceil(token_budget / 8) per row, rounded up to 256 bytes; tagged score
 * partials [batch_rows, max_chunks, num_kv_heads] x 8 bytes).  A workspace
 * serves one launch at a time.  Word 2 of its header is the owner's status
 * word: 0 unless a bounded wait of a single launch expired since the owner
 * last cleared it (then that launch's results are not valid); each launch
 * ORs its own bits in when it ends and never clears it.
 */
size_t ds_step_workspace_bytes(int batch_rows, int max_chunks, int num_kv_heads, int token_budget);

/*
 * The retrieval step with its scratch memory in a static device array.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * allocation).  Same work and results as ds_retrieval_step; the descriptor's
 * score_partials, workspace (and workspace_bytes) and lse_partials must be
 * NULL / 0, since those buffers live in a file-scope __device__ array of
 * DS_STATIC_SCRATCH_BYTES that each GPU holds from library load until the
 * process ends.  Every other buffer (inputs, outputs, per-slot state) is the
 * caller's, as before.  Nothing is allocated and no allocating routine is
 * called.
 *
 * Limits, rejected with DS_ERR_INVALID and a message:
 *   DS_STAGE_SELECT only together with DS_STAGE_SCORE (the selection reads
 *   partials that only the same call's scoring writes into the array);
 *   batch_rows x max_chunks x num_kv_heads x 4 bytes <= DS_STATIC_PARTIALS_BYTES;
 *   without an LSE, batch_rows x num_q_heads x max_chunks x 8 bytes <= DS_STATIC_PAIRS_BYTES.
 * A full step runs as the single launch when ds_step_workspace_bytes() of its
 * shape fits DS_STATIC_FUSED_BYTES (and the shape suits it), else as the chain.
 * status (optional, a device word the caller owns and clears): a single
 * launch whose bounded wait expired ORs its status bits into it (then that
 * call's results are not valid).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (several streams or threads) race and must be serialised by the
 * caller.  The current device must be the stream's device.
 */
#define DS_STATIC_FUSED_BYTES ((size_t)8 << 20)
#define DS_STATIC_PARTIALS_BYTES ((size_t)4 << 20)
#define DS_STATIC_PAIRS_BYTES ((size_t)12 << 20)
#define DS_STATIC_SCRATCH_BYTES (DS_STATIC_FUSED_BYTES + DS_STATIC_PARTIALS_BYTES + DS_STATIC_PAIRS_BYTES)

int ds_retrieval_step_static(ds_stream_t stream, const ds_step_desc* desc, uint32_t* status);

/*
 * Draft decode attention over the working cache (linear drafting, one query
 * token per row).
 * Replaces DiffSpecDraftCache.forward_attention's linear path
 * (diffspec/runtime.py:2024-2077 on the CPU, and the batched
 * npu_fused_infer_attention_score call over the capacity view with
 * actual_seq_lengths_kv = position + 1, diffspec/runtime.py:2079-2134).
 *
 * For every row r < rows, with s = slots[r] and
 * p = positions ? positions[r] : working_lens[s] (read before this call
 * changes it):
 *   working_key[s, h, p] = key[r, h]; working_value[s, h, p] = value[r, h]
 *   working_lens[s] = p + 1
 *   out[r, hq] = sum_t softmax_t(scale * q[r, hq] . K[s, hq / G, t]) V[s, hq / G, t],
 *                t = 0..p, G = num_q_heads / num_kv_heads (query head hq
 *                uses KV head hq / G, the reference's repeat_interleave),
 *                scores, softmax and the weighted sum in fp32, rounded once
 *                to the output dtype;
 * rows rows <= r < out_rows of `out` are written as zeros (the reference's
 * output.zero_() for graph padding).  A row whose slot or position is out
 * of range ([0, num_slots), [0, token_budget)) gets zeros, changes nothing
 * else and sets bit 0 of the workspace status word (the reference raises
 * "DiffSpec working cache exhausted" on the host).
 *
 * query  : [out_rows, Hq, D]   element (r, h, d) at r*q_row_stride + h*q_head_stride + d
 * key, value: [rows, Hkv, D]   (new token's K/V, same addressing)
 * out    : [out_rows, Hq, D]
 * working_key / working_value: [num_slots, Hkv, token_budget, D] contiguous
 * working_lens: int32 [num_slots]; slots, positions: int32 [rows]
 * dtype  : DS_BF16 or DS_FP16 for every tensor; head_dim 64, 128 or 256;
 *          row and head strides multiples of 8 elements, 16-byte aligned
 *          pointers.
 * workspace: zero-filled once, >= ds_draft_attention_workspace_bytes(),
 *          256-byte aligned; reused across launches (one stream at a time).
 *          Word 2 of its header is the status word (bit 1: the wait of the
 *          last workgroup for the others' "seen" words expired: that
 *          launch's working lengths were not advanced).
 * One kernel launch, no host synchronisation, fixed launch shape for the
 * given sizes (graph-capturable).
 */
int ds_draft_attention(ds_stream_t stream, int dtype,
                       const void* query, int64_t q_row_stride, int64_t q_head_stride,
                       const void* key, int64_t k_row_stride, int64_t k_head_stride,
                       const void* value, int64_t v_row_stride, int64_t v_head_stride,
                       void* out, int64_t o_row_stride, int64_t o_head_stride,
                       void* working_key, void* working_value, int32_t* working_lens,
                       const int32_t* slots, const int32_t* positions,
                       int rows, int out_rows, int num_slots,
                       int num_q_heads, int num_kv_heads, int head_dim, int token_budget,
                       float scale, void* workspace, size_t workspace_bytes);

/*
 * Workspace bytes of ds_draft_attention for up to batch_rows rows (0 when
 * an argument is not positive or Hq is not a multiple of Hkv).  No reference
 * counterpart.  With U = batch_rows x Hkv x ceil(G / 16) row units (at most
 * 65536) and W = U x ceil(token_budget / span) workgroups (span = 256
 * tokens, 128 for head_dim 256): 256 header bytes (word 0 the epoch, word 2
 * the status), 65536 4-byte span counters (0 between launches, at a fixed
 * place for every shape), W 8-byte tagged "seen" words rounded up to 256
 * bytes, then W x 16 x (head_dim + 4) fp32 partial results.
 */
size_t ds_draft_attention_workspace_bytes(int batch_rows, int num_q_heads, int num_kv_heads, int head_dim,
                                          int token_budget);

/*
 * Raw pre-RoPE K/V capture of draft tokens and the graph-safe RoPE input,
 * in one launch.
 * Replaces DiffSpecDraftCache._write_raw (diffspec/runtime.py:1602-1618), the
 * local positions of capture_raw_kv (diffspec/runtime.py:1797-1877) and
 * graph_safe_rope_positions (diffspec/runtime.py:1767-1794), which the
 * reference runs as torch index ops over index tensors built on the host
 * (the vllm::diffspec_capture_raw_kv op, diffspec/vllm_patch.py:132-178).
 *
 *   token t < tokens:  raw_key[token_slots[t], positions[t], h, :] = key[t, h, :]
 *                      raw_value likewise, every KV head h;
 *   rope_positions[t], t < count:
 *       working_lens given   : t < tokens ? working_lens[token_slots[t]] : 0
 *                              (draft rows at their local positions, graph
 *                              padding 0);
 *       local_positions given: local_positions[t];
 *       neither              : positions[t];
 *   rope_positions[t] = 0 for count <= t < prev_count (the previous call's
 *                              stale tail).
 * tokens <= count, or count == 0: the scatter alone, with no RoPE input
 * (DiffSpecDraftCache.populate_prefill, diffspec/runtime.py:1336-1347,
 * which writes the draft's projected prefill rows, rejected ones included).
 * positions, local_positions and rope_positions are int32, or int64 when
 * positions_int64 != 0.  key/value rows: element (t, h, d) at
 * t * row_stride + h * head_stride + d.  raw caches: [num_slots,
 * max_model_len, heads, head_dim] contiguous.  dtype: DS_BF16/FP16/FP32
 * (rows that are whole, aligned 16-byte vectors move as vectors, others
 * element by element).
 * A token whose slot or position is out of range is not written and sets
 * bit 0 of *status (status may be NULL).  One launch.
 */
int ds_capture_raw_kv(ds_stream_t stream, int dtype,
                      const void* key, int64_t k_row_stride, int64_t k_head_stride,
                      const void* value, int64_t v_row_stride, int64_t v_head_stride,
                      const void* positions, int positions_int64,
                      const int32_t* token_slots, int tokens,
                      void* raw_key, void* raw_value,
                      int num_slots, int max_model_len, int heads, int head_dim,
                      const int32_t* working_lens, const void* local_positions,
                      void* rope_positions, int count, int prev_count, int32_t* status);

#ifdef __cplusplus
}
#endif
#endif /* DS355_H */
