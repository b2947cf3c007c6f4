// Per-row top-k chunk selection and history-plan construction.
//
// Selection counterpart of diffspec/runtime.py:348-414 (called per row from
// runtime.py:1298-1308); plan counterpart of runtime.py:1713-1757.  One
// 256-thread workgroup per row:
//   1. scores -> order-preserving uint32 keys in LDS (larger key = better;
//      NaN ranks highest and -0 equals +0, as torch's sort treats them);
//   2. 4-pass MSB radix select (256-bin LDS histograms, block scan over the
//      bins) finds the (K-1)-th largest key T of chunks 0..C-2;
//   3. one ordered pass over the candidates keeps keys > T and the first
//      ties == T by index, compacting with block-wide exclusive scans, so the
//      ids come out ascending with no sort; the newest chunk C-1 is appended;
//   4. the plan row [slot, history_len, tail_start, prefix_len, prefix_drop,
//      chunk ids..., 0...] is built from the slot's selection in the same
//      workgroup (block reduction for prefix_tokens).
#include "select_body.h"

namespace ds355 {
namespace {

using namespace select;

constexpr int kLdsKeys = 12288;  // candidates kept in LDS; larger rows read keys from global memory
constexpr int kPre = 4;          // chunks per thread whose partials are loaded at kernel start
constexpr int kMore = 12;        // chunks per thread per later round (longer rows: 4096 chunks in two rounds)
constexpr int kLongRow = 2048;   // chunks per row from which the 1024-thread workgroup selects
constexpr int kLongThreads = 1024;

template <int HKV, int NT>
__global__ __launch_bounds__(NT) void select_plan_kernel(SelectArgs a) {
  __shared__ SelectShared<kLdsKeys, NT> sh;

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  // Every independent load is issued here, before any is waited for: the
  // row description, the slot, the committed length, the slot's stored
  // selection count (slots of distinct rows are distinct, so no other
  // workgroup writes counts[slot] in this launch) and the score partials of
  // the row's first kPre * 256 chunks (clamped to the buffer; masked below).
  const RowDesc d = a.do_select ? row_desc(a.src, b) : RowDesc{0, 0, 0};
  const int slot = a.slots != nullptr ? a.slots[b] : b;
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  int committed = a.do_plan ? committed_of(a.committed_lens, a.src, b) : 0;
  int stored_count = (a.do_plan && slot_ok) ? a.counts[slot] : 0;
  int32_t gen0 = (a.gen != nullptr && a.do_select && slot_ok) ? a.gen[slot] : 0;
  const float* part = a.partials + static_cast<int64_t>(b) * a.max_chunks * a.hkv;
  float pre[kPre];
  if (a.do_select && a.partials != nullptr) {
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int i = min(u * NT + tid, a.max_chunks - 1);
      pre[u] = head_sum<HKV>(part + static_cast<int64_t>(i) * a.hkv, a.hkv);
    }
  }
  // Made scalar (waited for) here, behind the loads above: they are used
  // only after the selection's stores, where waiting for their loads would
  // wait for those stores too.
  committed = __builtin_amdgcn_readfirstlane(committed);
  stored_count = __builtin_amdgcn_readfirstlane(stored_count);
  gen0 = __builtin_amdgcn_readfirstlane(gen0);
  int n_sel = -1;  // selection made by this workgroup (in sh.ids), -1 if none

  if (a.do_select && d.active && slot_ok) {
    const int C = (d.len + a.chunk - 1) / a.chunk;
    const int K = a.budget / a.chunk;
    if (C <= K) {
      for (int i = tid; i < C; i += NT) sh.ids[i] = i;
      n_sel = C;
    }
    float* row_scores = a.scores + static_cast<int64_t>(b) * a.score_stride;
    const int N = C - 1;  // candidates (newest chunk excluded from the ranking)
    const bool in_lds = C > K && N <= kLdsKeys;
    // Bounds of the candidate keys this thread computes (for select_top).
    uint32_t kmin = ~0u, kmax = 0u;
    const bool bounded = a.partials != nullptr || in_lds;
    if (a.partials != nullptr) {
      auto finish = [&](int i, float sum) {
        const float v = chunk_score(sum, a.chunk, d.len, i, a.hq);
        row_scores[i] = v;
        if (i < N) {
          const uint32_t key = order_key(v);
          kmin = min(kmin, key);
          kmax = max(kmax, key);
          if (in_lds) sh.keys[i] = key;
        }
      };
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int i = u * NT + tid;
        if (i < C) finish(i, pre[u]);
      }
      // Longer rows: kMore chunks per thread at a time, their loads issued
      // together (clamped to the buffer, masked when finished).
      for (int i0 = kPre * NT; i0 < C; i0 += kMore * NT) {
        float v[kMore];
#pragma unroll
        for (int u = 0; u < kMore; ++u) {
          const int i = min(i0 + u * NT + tid, a.max_chunks - 1);
          v[u] = head_sum<HKV>(part + static_cast<int64_t>(i) * a.hkv, a.hkv);
        }
#pragma unroll
        for (int u = 0; u < kMore; ++u) {
          const int i = i0 + u * NT + tid;
          if (i < C) finish(i, v[u]);
        }
      }
    } else if (in_lds) {
      for (int i = tid; i < N; i += NT) {
        const uint32_t key = order_key(row_scores[i]);
        kmin = min(kmin, key);
        kmax = max(kmax, key);
        sh.keys[i] = key;
      }
    }
    if (in_lds) {
      lds_barrier();
    } else {
      __syncthreads();  // keys are read back from the score row in global memory
    }
    if (C > K) {
      select_top(sh, N, K, [&](int q) -> U4 {
        if (in_lds) return *reinterpret_cast<const U4*>(&sh.keys[4 * q]);
        U4 k4;
#pragma unroll
        for (int j = 0; j < 4; ++j) k4[j] = order_key(row_scores[min(4 * q + j, N - 1)]);
        return k4;
      }, bounded ? kmin : 0u, bounded ? kmax : ~0u);
      n_sel = K;
    }
    lds_barrier();
    int32_t* out = a.ids + static_cast<int64_t>(slot) * a.ids_stride;
    for (int j = tid; j < n_sel; j += NT) out[j] = sh.ids[j];
    if (tid == 0) {
      a.counts[slot] = n_sel;
      if (a.gen != nullptr) a.gen[slot] = gen0 + 1;  // one row per slot: no other writer
    }
  }

  if (!a.do_plan) return;
  if (!slot_ok) {
    int64_t* prow = a.plan + static_cast<int64_t>(b) * a.plan_width;
    for (int j = tid; j < a.plan_width; j += NT) prow[j] = 0;
    return;
  }
  write_plan_row(a, b, slot, committed, n_sel, stored_count, sh);
}

}  // namespace

int make_select_args(SelectArgs& a, float* scores, int64_t score_stride, const float* partials, int max_chunks,
                     int hkv, int hq, const RowSource& src, int batch, int chunk, int budget, int do_select,
                     int do_plan, int32_t* ids, int64_t ids_stride, int32_t* counts, const int32_t* slots,
                     int num_slots, const int32_t* committed_lens, int64_t* plan, int plan_width,
                     int32_t* working_lens, int recent_window) {
  a = SelectArgs{};
  DS_REQUIRE(chunk > 0, "chunk_size must be positive");
  DS_REQUIRE(budget >= chunk && budget % chunk == 0, "token_budget must be a positive chunk-size multiple");
  DS_SUPPORTED(budget / chunk <= kMaxSel, "at most %d selected chunks (got %d)", kMaxSel, budget / chunk);
  DS_REQUIRE(batch >= 0, "batch must be non-negative");
  DS_SUPPORTED(batch <= 65535, "at most 65535 rows per launch");
  if (do_select) DS_REQUIRE(ids_stride >= budget / chunk, "selection row stride is smaller than the chunk capacity");
  if (do_plan) {
    DS_REQUIRE(plan_width >= 5 + budget / chunk, "plan width is smaller than 5 + history_budget / chunk_size");
    DS_REQUIRE(recent_window > 0, "recent_window must be positive");
  }
  if (batch == 0) return clear_error();
  if (do_select) DS_REQUIRE(scores && ids && counts && (src.seq_lens || src.counts), "null selection pointer");
  if (do_plan) DS_REQUIRE(ids && counts && plan && (committed_lens || src.counts), "null plan pointer");

  if (do_select && partials != nullptr) DS_REQUIRE(hkv > 0 && hq > 0 && max_chunks > 0, "bad score partial shape");
  a.scores = scores;
  a.score_stride = score_stride;
  a.partials = partials;
  a.max_chunks = max_chunks;
  a.hkv = hkv;
  a.hq = hq;
  a.src = src;
  a.batch = batch;
  a.chunk = chunk;
  a.budget = budget;
  a.do_select = do_select;
  a.do_plan = do_plan;
  a.ids = ids;
  a.ids_stride = ids_stride;
  a.counts = counts;
  a.slots = slots;
  a.num_slots = num_slots;
  a.committed_lens = committed_lens;
  a.plan = plan;
  a.plan_width = plan_width;
  a.working_lens = working_lens;
  a.recent_window = recent_window;
  return clear_error();
}

namespace {
template <int NT>
int launch_hkv(hipStream_t stream, const SelectArgs& a, int hkv, int batch) {
  switch (hkv) {
    case 1: select_plan_kernel<1, NT><<<batch, NT, 0, stream>>>(a); break;
    case 2: select_plan_kernel<2, NT><<<batch, NT, 0, stream>>>(a); break;
    case 4: select_plan_kernel<4, NT><<<batch, NT, 0, stream>>>(a); break;
    case 8: select_plan_kernel<8, NT><<<batch, NT, 0, stream>>>(a); break;
    default: select_plan_kernel<0, NT><<<batch, NT, 0, stream>>>(a); break;
  }
  return check_launch("select/plan");
}
}  // namespace

int launch_select_plan(hipStream_t stream, float* scores, int64_t score_stride, const float* partials,
                       int max_chunks, int hkv, int hq, const RowSource& src,
                       int batch, int chunk, int budget, int do_select, int do_plan, int32_t* ids,
                       int64_t ids_stride, int32_t* counts, const int32_t* slots, int num_slots,
                       const int32_t* committed_lens, int64_t* plan, int plan_width, int32_t* working_lens,
                       int recent_window, int32_t* gen) {
  SelectArgs a;
  const int rc = make_select_args(a, scores, score_stride, partials, max_chunks, hkv, hq, src, batch, chunk, budget,
                                  do_select, do_plan, ids, ids_stride, counts, slots, num_slots, committed_lens, plan,
                                  plan_width, working_lens, recent_window);
  if (rc != DS_OK || batch == 0) return rc;
  a.gen = gen;
  // Rows of kLongRow chunks or more are selected by 1024-thread workgroups
  // (four times the waves for the per-candidate sweeps), shorter ones by 256.
  const int64_t row_chunks = (static_cast<int64_t>(src.max_len) + chunk - 1) / chunk;
  if (do_select && row_chunks >= kLongRow) return launch_hkv<kLongThreads>(stream, a, partials != nullptr ? hkv : 0, batch);
  return launch_hkv<kThreads>(stream, a, do_select && partials != nullptr ? hkv : 0, batch);
}

}  // namespace ds355

extern "C" int ds_select_chunks(ds_stream_t stream, const float* scores, int64_t score_stride, int score_cols,
                                const int32_t* seq_lens, int batch, int chunk_size, int history_budget,
                                int32_t* ids, int64_t ids_stride, int32_t* counts) {
  DS_REQUIRE(chunk_size > 0, "chunk_size must be positive");
  DS_REQUIRE(score_cols >= 0 && score_cols <= score_stride, "score_cols must be between 0 and the row stride");
  ds355::RowSource src{};
  src.seq_lens = seq_lens;
  src.max_len = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(score_cols) * chunk_size, INT32_MAX));
  return ds355::launch_select_plan(reinterpret_cast<hipStream_t>(stream), const_cast<float*>(scores), score_stride,
                                   nullptr, 0, 0, 0, src, batch,
                                   chunk_size, history_budget, 1, 0, ids, ids_stride, counts, nullptr, batch,
                                   nullptr, nullptr, 0, nullptr, chunk_size, nullptr);
}

extern "C" int ds_build_plan(ds_stream_t stream, const int32_t* sel_ids, int64_t sel_stride,
                             const int32_t* sel_count, int num_slots, const int32_t* slots,
                             const int32_t* committed_lens, int rows,
                             int chunk_size, int history_budget, int recent_window, int64_t* plan, int plan_width,
                             int32_t* working_lens) {
  if (rows > 0) DS_REQUIRE(slots != nullptr, "null slots pointer");
  DS_REQUIRE(num_slots > 0, "num_slots must be positive");
  ds355::RowSource src{};
  src.max_len = 0;
  return ds355::launch_select_plan(reinterpret_cast<hipStream_t>(stream), nullptr, 0, nullptr, 0, 0, 0, src, rows,
                                   chunk_size,
                                   history_budget, 0, 1, const_cast<int32_t*>(sel_ids), sel_stride,
                                   const_cast<int32_t*>(sel_count), slots, num_slots, committed_lens, plan,
                                   plan_width, working_lens, recent_window, nullptr);
}
