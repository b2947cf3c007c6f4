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
#include "rowdesc.h"

namespace ds355 {
namespace {

constexpr int kThreads = 256;
constexpr int kLdsKeys = 12288;  // candidates kept in LDS; larger rows read keys from global memory
constexpr int kMaxSel = 2048;    // chunk ids per selection
constexpr int kPre = 4;          // chunks per thread whose partials are loaded at kernel start

struct SelectArgs {
  float* scores;           // final scores [batch, score_stride]; written here when partials are given
  int64_t score_stride;
  const float* partials;   // per-KV-head sums [batch, max_chunks, hkv] from the score pass, or nullptr
  int max_chunks, hkv, hq;
  RowSource src;
  int batch;
  int chunk;
  int budget;  // history budget (multiple of chunk)
  int do_select;
  int do_plan;
  int32_t* ids;  // selection output / state, row = slot (or b without slots)
  int64_t ids_stride;
  int32_t* counts;
  const int32_t* slots;  // nullptr: row b writes selection row b
  const int32_t* committed_lens;
  int64_t* plan;
  int plan_width;
  int32_t* working_lens;
  int recent_window;
  int num_slots;
};

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN: largest
  if ((u & 0x7fffffffu) == 0u) u = 0u;                      // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Workgroup barrier for LDS hand-offs only.  Unlike __syncthreads it does
// not wait for this wave's outstanding global stores (the score row), which
// other kernels read and this workgroup does not.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Exclusive scan over the 256 threads through LDS; `total` gets the sum.
__device__ __forceinline__ int lds_exclusive_scan(int v, int* scratch, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int inc = wave_inclusive_scan(v);
  if (lane == 63) scratch[wave] = inc;
  lds_barrier();
  int base = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    const int t = scratch[w];
    if (w < wave) base += t;
    total += t;
  }
  lds_barrier();
  return base + inc - v;
}

__device__ __forceinline__ int block_inclusive_scan(int v, int* scratch) {
  int total;
  return lds_exclusive_scan(v, scratch, total) + v;
}

__device__ __forceinline__ int block_sum(int v, int* scratch) {
  int total;
  lds_exclusive_scan(v, scratch, total);
  return total;
}

// Sum of one chunk's per-KV-head partials in head order (HKV == 0: runtime
// count); the HKV loads are unconditional and issued together.
template <int HKV>
__device__ __forceinline__ float head_sum(const float* pp, int hkv) {
  float sum = 0.f;
  if constexpr (HKV > 0) {
    float v[HKV];
#pragma unroll
    for (int g = 0; g < HKV; ++g) v[g] = pp[g];
#pragma unroll
    for (int g = 0; g < HKV; ++g) sum += v[g];
  } else {
    for (int g = 0; g < hkv; ++g) sum += pp[g];
  }
  return sum;
}

template <int HKV>
__global__ __launch_bounds__(kThreads) void select_plan_kernel(SelectArgs a) {
  __shared__ uint32_t s_keys[kLdsKeys];
  __shared__ int s_hist[256];
  __shared__ int s_ids[kMaxSel];
  __shared__ int s_scratch[4];
  __shared__ int s_digit, s_above, s_eq;

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
  const int committed = a.do_plan ? a.committed_lens[b] : 0;
  const int stored_count = (a.do_plan && slot_ok) ? a.counts[slot] : 0;
  const float* part = a.partials + static_cast<int64_t>(b) * a.max_chunks * a.hkv;
  float pre[kPre];
  if (a.do_select && a.partials != nullptr) {
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int i = min(u * kThreads + tid, a.max_chunks - 1);
      pre[u] = head_sum<HKV>(part + static_cast<int64_t>(i) * a.hkv, a.hkv);
    }
  }
  int n_sel = -1;  // selection made by this workgroup (in s_ids), -1 if none

  if (a.do_select && d.active && slot_ok) {
    const int C = (d.len + a.chunk - 1) / a.chunk;
    const int K = a.budget / a.chunk;
    if (C <= K) {
      for (int i = tid; i < C; i += kThreads) s_ids[i] = i;
      n_sel = C;
    }
    float* row_scores = a.scores + static_cast<int64_t>(b) * a.score_stride;
    const int N = C - 1;  // candidates (newest chunk excluded from the ranking)
    const bool in_lds = C > K && N <= kLdsKeys;
    if (a.partials != nullptr) {
      // Final scores from the per-KV-head partials (fixed head order):
      // sum_g / n_valid / Hq, the same rounding steps as the drop-in finalize.
      auto finish = [&](int i, float sum) {
        const int n_valid = min(a.chunk, d.len - i * a.chunk);
        const float v = (sum / static_cast<float>(n_valid)) / static_cast<float>(a.hq);
        row_scores[i] = v;
        if (in_lds && i < N) s_keys[i] = order_key(v);
      };
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int i = u * kThreads + tid;
        if (i < C) finish(i, pre[u]);
      }
      for (int i = kPre * kThreads + tid; i < C; i += kThreads) {
        finish(i, head_sum<HKV>(part + static_cast<int64_t>(i) * a.hkv, a.hkv));
      }
    } else if (in_lds) {
      for (int i = tid; i < N; i += kThreads) s_keys[i] = order_key(row_scores[i]);
    }
    if (in_lds) {
      lds_barrier();
    } else {
      __syncthreads();  // keys are read back from the score row in global memory
    }
    if (C > K) {
      int need = K - 1;
      auto key_at = [&](int i) -> uint32_t { return in_lds ? s_keys[i] : order_key(row_scores[i]); };

      uint32_t prefix = 0u, pmask = 0u;
      bool take_all_ties = true;
      if (need > 0) {
        for (int shift = 24; shift >= 0; shift -= 8) {
          s_hist[tid] = 0;
          lds_barrier();
          for (int i = tid; i < N; i += kThreads) {
            const uint32_t k = key_at(i);
            if ((k & pmask) == prefix) atomicAdd(&s_hist[(k >> shift) & 0xffu], 1);
          }
          lds_barrier();
          const int digit = 255 - tid;  // thread t scans bins in descending digit order
          const int cnt = s_hist[digit];
          const int incl = block_inclusive_scan(cnt, s_scratch);
          if (incl - cnt < need && need <= incl) {
            s_digit = digit;
            s_above = incl - cnt;
            s_eq = cnt;
          }
          lds_barrier();
          prefix |= static_cast<uint32_t>(s_digit) << shift;
          pmask |= 0xffu << shift;
          need -= s_above;
          if (shift == 0) take_all_ties = (need == s_eq);
          lds_barrier();
        }
      }
      // need = ties (key == T) still to take, lowest indices first.
      const uint32_t T = prefix;
      const bool none = (K - 1) == 0;
      int carry_sel = 0, carry_eq = 0;
      if (!none) {
        for (int base = 0; base < N; base += kThreads) {
          const int i = base + tid;
          const uint32_t k = i < N ? key_at(i) : 0u;
          const bool gt = i < N && k > T;
          const bool eq = i < N && k == T;
          bool sel;
          if (take_all_ties) {
            sel = gt || eq;
          } else {
            int eq_total;
            const int eq_ex = lds_exclusive_scan(eq ? 1 : 0, s_scratch, eq_total);
            sel = gt || (eq && carry_eq + eq_ex < need);
            carry_eq += eq_total;
          }
          int sel_total;
          const int sel_ex = lds_exclusive_scan(sel ? 1 : 0, s_scratch, sel_total);
          if (sel && carry_sel + sel_ex < kMaxSel) s_ids[carry_sel + sel_ex] = i;
          carry_sel += sel_total;
        }
      }
      if (tid == 0) s_ids[K - 1] = C - 1;
      n_sel = K;
    }
    lds_barrier();
    int32_t* out = a.ids + static_cast<int64_t>(slot) * a.ids_stride;
    for (int j = tid; j < n_sel; j += kThreads) out[j] = s_ids[j];
    if (tid == 0) a.counts[slot] = n_sel;
  }

  if (!a.do_plan) return;
  int64_t* prow = a.plan + static_cast<int64_t>(b) * a.plan_width;
  if (!slot_ok) {
    for (int j = tid; j < a.plan_width; j += kThreads) prow[j] = 0;
    return;
  }
  // The slot's selection: just made here, or the stored one.
  const int64_t cap = min(static_cast<int64_t>(a.plan_width - 5), a.ids_stride);
  const int count = n_sel >= 0 ? n_sel : static_cast<int>(min(static_cast<int64_t>(stored_count), cap));
  const int32_t* stored = a.ids + static_cast<int64_t>(slot) * a.ids_stride;
  auto chunk_id = [&](int j) -> int64_t { return n_sel >= 0 ? s_ids[j] : stored[j]; };

  const int64_t end = max(0, committed - 1);
  const int64_t hb = a.budget;
  int64_t len, tail_start, prefix_len = 0, drop = 0;
  int ncols = 0;
  if (count < 0) {
    len = min(end, hb);
    tail_start = end - len;
  } else {
    const int64_t tail_len = min(min(end, static_cast<int64_t>(a.recent_window)), hb);
    tail_start = end - tail_len;
    len = tail_len;
    if (count > 0) {
      ncols = min(count, a.plan_width - 5);
      const int64_t prefix_end = min(tail_start, chunk_id(count - 1) * a.chunk);
      int64_t part = 0;
      for (int j = tid; j < count; j += kThreads) {
        const int64_t t = prefix_end - chunk_id(j) * a.chunk;
        part += t <= 0 ? 0 : (t < a.chunk ? t : a.chunk);
      }
      // Block sum in int (each term <= chunk; the total <= count * chunk).
      const int64_t prefix_tokens = block_sum(static_cast<int>(part), s_scratch);
      prefix_len = min(prefix_tokens, hb - tail_len);
      drop = prefix_tokens - prefix_len;
      len = prefix_len + tail_len;
    }
  }
  for (int j = tid; j < a.plan_width; j += kThreads) {
    int64_t v;
    if (j == 0) v = slot;
    else if (j == 1) v = len;
    else if (j == 2) v = tail_start;
    else if (j == 3) v = prefix_len;
    else if (j == 4) v = drop;
    else v = (j - 5) < ncols ? chunk_id(j - 5) : 0;
    prow[j] = v;
  }
  if (tid == 0 && a.working_lens != nullptr) a.working_lens[slot] = static_cast<int32_t>(len);
}

}  // namespace

int launch_select_plan(hipStream_t stream, float* scores, int64_t score_stride, const float* partials,
                       int max_chunks, int hkv, int hq, const RowSource& src,
                       int batch, int chunk, int budget, int do_select, int do_plan, int32_t* ids,
                       int64_t ids_stride, int32_t* counts, const int32_t* slots, int num_slots,
                       const int32_t* committed_lens, int64_t* plan, int plan_width, int32_t* working_lens,
                       int recent_window) {
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
  if (do_plan) DS_REQUIRE(ids && counts && committed_lens && plan, "null plan pointer");

  if (do_select && partials != nullptr) DS_REQUIRE(hkv > 0 && hq > 0 && max_chunks > 0, "bad score partial shape");
  SelectArgs a{};
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
  switch (do_select && partials != nullptr ? hkv : 0) {
    case 1: select_plan_kernel<1><<<batch, kThreads, 0, stream>>>(a); break;
    case 2: select_plan_kernel<2><<<batch, kThreads, 0, stream>>>(a); break;
    case 4: select_plan_kernel<4><<<batch, kThreads, 0, stream>>>(a); break;
    case 8: select_plan_kernel<8><<<batch, kThreads, 0, stream>>>(a); break;
    default: select_plan_kernel<0><<<batch, kThreads, 0, stream>>>(a); break;
  }
  return check_launch("select/plan");
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
                                   nullptr, nullptr, 0, nullptr, chunk_size);
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
                                   plan_width, working_lens, recent_window);
}
