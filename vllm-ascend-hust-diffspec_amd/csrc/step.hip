// One retrieval step on one stream: the single-launch kernel (fused.hip)
// when the descriptor brings a workspace and fits it, otherwise a chain:
//   chunk_score_kernel (rows with committed tokens; committed query; rejected
//   suffix cut; without a softmax LSE, plus lse_finalize_kernel) ->
//   select_plan_kernel (selection into the per-slot state, then a plan row
//   for every real row) -> gather kernel over the plan.
// No host synchronisation; launch shapes depend only on the descriptor's
// upper bounds, so the chain can be captured into a HIP graph.
#include "rowdesc.h"

namespace ds355 {

int launch_chunk_scores(hipStream_t stream, int dtype, const void* query, int64_t q_stride, const void* key_cache,
                        int64_t k_block_stride, int64_t k_token_stride, int64_t k_head_stride, const float* lse,
                        int64_t lse_row_stride, int64_t lse_head_stride, const int32_t* block_table,
                        int64_t bt_stride, const RowSource& src, int batch, int num_q_heads, int num_kv_heads,
                        int head_dim, int block_size, int chunk_size, int max_chunks, float scale, int head_reduce,
                        float* partial, float* out, int64_t out_stride, int write_tail, size_t partial_bytes,
                        uint64_t* mw, float* lse_out, int64_t lse_out_stride);

int launch_select_plan(hipStream_t stream, float* scores, int64_t score_stride, const float* partials,
                       int max_chunks, int hkv, int hq, const RowSource& src,
                       int batch, int chunk, int budget, int do_select, int do_plan, int32_t* ids,
                       int64_t ids_stride, int32_t* counts, const int32_t* slots, int num_slots,
                       const int32_t* committed_lens, int64_t* plan, int plan_width, int32_t* working_lens,
                       int recent_window, int32_t* gen);

int rebuild_compact_kv_impl(hipStream_t stream, int dtype, const void* raw_key, const void* raw_value,
                            void* working_key, void* working_value, const int64_t* plan, int rows,
                            int plan_width, const void* cos_sin, int64_t cs_stride, int cs_rows, int num_slots,
                            int max_model_len, int heads, int head_dim, int token_budget, int chunk_size,
                            int rotary_dim, int is_neox_style, int max_width, const int32_t* row_active,
                            bool padded_rows);

int launch_fused_step(hipStream_t stream, const ds_step_desc* d, const RowSource& src, uint32_t* status_out,
                      bool& launched);

int launch_plan_gather(hipStream_t stream, int dtype, const void* raw_key, const void* raw_value,
                       void* working_key, void* working_value, int rows, int plan_width, const void* cos_sin,
                       int64_t cs_stride, int cs_rows, int num_slots, int max_model_len, int heads, int head_dim,
                       int token_budget, int chunk_size, int rotary_dim, int is_neox_style, int history_budget,
                       const int32_t* row_active, const int32_t* sel_ids, int64_t sel_stride,
                       const int32_t* sel_count, const int32_t* slots, const int32_t* committed_lens, int64_t* plan,
                       int32_t* working_lens, int recent_window, const int32_t* gen, uint64_t* rec,
                       int64_t rec_stride, bool prefix_only, const RowSource& src, bool& launched);

int clear_gather_records(hipStream_t stream, const int32_t* slots, int rows, int num_slots,
                         const int32_t* row_active, uint64_t* rec, int64_t rec_stride, int64_t entries);

// The step for a descriptor whose scratch buffers are already set.
// status_out (optional): a single launch ORs its status bits into it.
int retrieval_step(hipStream_t stream, const ds_step_desc* d, uint32_t* status_out) {
  DS_REQUIRE(d != nullptr, "null step descriptor");
  DS_REQUIRE((d->stages & ~(DS_STAGE_ALL | DS_STAGE_PREFIX)) == 0, "unknown stage bits 0x%x", d->stages);
  const bool score = (d->stages & DS_STAGE_SCORE) != 0;
  const bool select = (d->stages & DS_STAGE_SELECT) != 0;
  const bool full = (d->stages & DS_STAGE_PLAN) != 0;
  const bool prefix = !full && (d->stages & DS_STAGE_PREFIX) != 0;
  const bool rebuild = full || prefix;
  const bool records = d->gather_rec != nullptr;
  // A prefix-only rebuild leaves the working lengths to the compact prefill.
  int32_t* const working_lens = prefix ? nullptr : d->working_lens;
  DS_REQUIRE(records == (d->sel_gen != nullptr), "sel_gen and gather_rec come together");
  DS_REQUIRE(!prefix || records, "DS_STAGE_PREFIX needs gather records (sel_gen, gather_rec)");
  // The prefix stage reads each row's verifier rows (which raw rows the
  // draft's prefill rewrites): it comes with the selection, in the retrieval call.
  DS_REQUIRE(!prefix || select, "DS_STAGE_PREFIX runs with DS_STAGE_SELECT (it needs the verifier rows)");
  if (records) DS_REQUIRE(d->rec_stride >= d->token_budget, "gather record row stride is smaller than token_budget");
  DS_REQUIRE(!rebuild || d->committed_lens != nullptr || prefix,
             "the plan needs committed_lens (or, for DS_STAGE_PREFIX, the verifier rows)");
  DS_REQUIRE(d->batch_rows >= 0 && d->batch_size >= 0 && d->batch_size <= d->batch_rows,
             "batch_size must be between zero and batch_rows");
  DS_REQUIRE(d->chunk_size > 0 && d->history_budget >= d->chunk_size && d->history_budget % d->chunk_size == 0,
             "history_budget must be a positive chunk-size multiple");
  DS_REQUIRE(d->history_budget < d->token_budget, "history_budget must be smaller than token_budget");
  DS_REQUIRE(d->plan_width == 5 + d->token_budget / d->chunk_size, "plan width must be 5 + working_budget // chunk_size");
  DS_REQUIRE(d->sel_stride >= d->token_budget / d->chunk_size, "selection row stride is smaller than the plan capacity");
  if (d->batch_rows == 0 || d->stages == 0) return clear_error();

  RowSource src{};
  src.counts = d->counts;
  src.q_start = d->query_start;
  src.q_len = d->query_len;
  src.target_len = d->target_len;
  src.batch_size = d->batch_size;
  if (score || select) {
    DS_REQUIRE(d->counts && d->query_start && d->query_len && d->target_len, "null verifier row pointer");
    DS_REQUIRE(d->max_chunks > 0 && d->scores != nullptr && d->score_partials != nullptr,
               "score and score-partial buffers are required");
    DS_REQUIRE(d->num_kv_heads > 0 && d->num_q_heads > 0, "head counts must be positive");
  }
  if (score) {
    DS_REQUIRE(d->lse != nullptr || (d->lse_partials != nullptr && d->lse_out != nullptr),
               "without a softmax LSE the step needs lse_partials ([batch_rows, max_chunks, Hq, 2] fp32) and "
               "lse_out ([batch_rows, Hq] fp32)");
  }
  src.max_len = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(d->max_chunks) * d->chunk_size, INT32_MAX));
  bool launched = false;
  int rc = launch_fused_step(stream, d, src, status_out, launched);
  if (rc != DS_OK || launched) return rc;
  if (score) {
    rc = launch_chunk_scores(stream, d->dtype, d->query, d->q_stride, d->key_cache, d->k_block_stride,
                             d->k_token_stride, d->k_head_stride, d->lse, d->lse_token_stride, d->lse_head_stride,
                             d->block_table, d->bt_stride, src, d->batch_rows, d->num_q_heads, d->num_kv_heads,
                             d->head_dim, d->block_size, d->chunk_size, d->max_chunks, d->scale, DS_HEAD_MEAN,
                             d->score_partials, nullptr, 0, 0, SIZE_MAX, reinterpret_cast<uint64_t*>(d->lse_partials), d->lse_out,
                             d->lse_out_stride);
    if (rc != DS_OK) return rc;
  }
  // The rebuild as one plan + gather launch (the compact prefill's kernel)
  // when the gather's vector path covers the shapes and nothing needs the
  // plan kernel's selection: always alone, and after a selection when the
  // gather keeps records.
  if (rebuild && (!select || records)) {
    if (select) {
      rc = launch_select_plan(stream, d->scores, d->max_chunks, d->score_partials, d->max_chunks, d->num_kv_heads,
                              d->num_q_heads, src, d->batch_rows, d->chunk_size, d->history_budget, 1, 0,
                              d->sel_ids, d->sel_stride, d->sel_count, d->slots, d->num_slots, d->committed_lens,
                              d->plan, d->plan_width, working_lens, d->recent_window, d->sel_gen);
      if (rc != DS_OK) return rc;
    }
    bool one = false;
    rc = launch_plan_gather(stream, d->kv_dtype, d->raw_key, d->raw_value, d->working_key, d->working_value,
                            d->batch_rows, d->plan_width, d->cos_sin, d->cs_stride, d->cs_rows, d->num_slots,
                            d->max_model_len, d->draft_heads, d->draft_head_dim, d->token_budget, d->chunk_size,
                            d->rotary_dim, d->is_neox_style, d->history_budget, d->row_active, d->sel_ids,
                            d->sel_stride, d->sel_count, d->slots, d->committed_lens, d->plan, working_lens,
                            d->recent_window, d->sel_gen, d->gather_rec, d->rec_stride, prefix, src, one);
    if (rc != DS_OK || one) return rc;
    // Shapes the one-launch rebuild does not cover: the plan kernel, then
    // (not for a prefix-only rebuild) the gather below moves every
    // position, and the records are cleared.
    if (records) {
      DS_REQUIRE(d->slots != nullptr, "gather records need the slots of the plan rows");
      rc = clear_gather_records(stream, d->slots, d->batch_rows, d->num_slots, d->row_active, d->gather_rec,
                                d->rec_stride, d->token_budget);
      if (rc != DS_OK) return rc;
    }
    rc = launch_select_plan(stream, d->scores, d->max_chunks, d->score_partials, d->max_chunks, d->num_kv_heads,
                            d->num_q_heads, src, d->batch_rows, d->chunk_size, d->history_budget, 0, 1, d->sel_ids,
                            d->sel_stride, d->sel_count, d->slots, d->num_slots, d->committed_lens, d->plan,
                            d->plan_width, working_lens, d->recent_window, nullptr);
    if (rc != DS_OK || prefix) return rc;
  } else if (select || rebuild) {
    rc = launch_select_plan(stream, d->scores, d->max_chunks, d->score_partials, d->max_chunks, d->num_kv_heads,
                            d->num_q_heads, src, d->batch_rows, d->chunk_size, d->history_budget,
                            select ? 1 : 0, rebuild ? 1 : 0, d->sel_ids, d->sel_stride, d->sel_count, d->slots,
                            d->num_slots, d->committed_lens, d->plan, d->plan_width, d->working_lens,
                            d->recent_window, d->sel_gen);
    if (rc != DS_OK) return rc;
  }
  if (!rebuild) return clear_error();
  return rebuild_compact_kv_impl(stream, d->kv_dtype, d->raw_key, d->raw_value, d->working_key, d->working_value,
                                 d->plan, d->batch_rows, d->plan_width, d->cos_sin, d->cs_stride, d->cs_rows,
                                 d->num_slots, d->max_model_len, d->draft_heads, d->draft_head_dim, d->token_budget,
                                 d->chunk_size, d->rotary_dim, d->is_neox_style, d->history_budget, d->row_active,
                                 true);
}

}  // namespace ds355

extern "C" int ds_retrieval_step(ds_stream_t stream, const ds_step_desc* d) {
  return ds355::retrieval_step(reinterpret_cast<hipStream_t>(stream), d, nullptr);
}
