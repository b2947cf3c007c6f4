// Per-row top-k selection and plan-row construction, shared by
// select_plan_kernel and the fused retrieval step.  See select_plan.hip for
// the algorithm.
#pragma once

#include "rowdesc.h"

namespace ds355 {
namespace select {

constexpr int kThreads = 256;
constexpr int kMaxSel = 2048;  // chunk ids per selection

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

// LDS of one selecting workgroup.  KEYS = candidates whose keys stay in LDS.
template <int KEYS>
struct SelectShared {
  uint32_t keys[KEYS];
  int hist[256];
  int ids[kMaxSel];
  int scratch[4];
  int digit, above, eq;
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

// Final chunk score from its head sum: sum_g / n_valid / Hq, the same
// rounding steps as the drop-in finalize.
__device__ __forceinline__ float chunk_score(float sum, int chunk, int len, int i, int hq) {
  const int n_valid = min(chunk, len - i * chunk);
  return (sum / static_cast<float>(n_valid)) / static_cast<float>(hq);
}

// Top K - 1 of the N candidates (chunks 0..N-1, keys from key_at) plus the
// newest chunk N, ascending, into sh.ids[0..K).  Starts and ends on a
// barrier-separated LDS state; requires N + 1 > K.
template <int KEYS, typename KeyAt>
__device__ __forceinline__ void select_top(SelectShared<KEYS>& sh, int N, int K, KeyAt key_at) {
  const int tid = threadIdx.x;
  int need = K - 1;
  uint32_t prefix = 0u, pmask = 0u;
  bool take_all_ties = true;
  if (need > 0) {
    for (int shift = 24; shift >= 0; shift -= 8) {
      sh.hist[tid] = 0;
      lds_barrier();
      for (int i = tid; i < N; i += kThreads) {
        const uint32_t k = key_at(i);
        if ((k & pmask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 0xffu], 1);
      }
      lds_barrier();
      const int digit = 255 - tid;  // thread t scans bins in descending digit order
      const int cnt = sh.hist[digit];
      const int incl = block_inclusive_scan(cnt, sh.scratch);
      if (incl - cnt < need && need <= incl) {
        sh.digit = digit;
        sh.above = incl - cnt;
        sh.eq = cnt;
      }
      lds_barrier();
      prefix |= static_cast<uint32_t>(sh.digit) << shift;
      pmask |= 0xffu << shift;
      need -= sh.above;
      if (shift == 0) take_all_ties = (need == sh.eq);
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
        const int eq_ex = lds_exclusive_scan(eq ? 1 : 0, sh.scratch, eq_total);
        sel = gt || (eq && carry_eq + eq_ex < need);
        carry_eq += eq_total;
      }
      int sel_total;
      const int sel_ex = lds_exclusive_scan(sel ? 1 : 0, sh.scratch, sel_total);
      if (sel && carry_sel + sel_ex < kMaxSel) sh.ids[carry_sel + sel_ex] = i;
      carry_sel += sel_total;
    }
  }
  if (tid == 0) sh.ids[K - 1] = N;
}

// Plan row of batch row b for a valid slot, from the selection just made
// (n_sel >= 0, ids in sh.ids) or the slot's stored one (n_sel < 0,
// stored_count entries).  Writes plan[b] (with device-scope stores when
// COHERENT) and working_lens[slot].  Contains barriers (block sum) when the
// selection is non-empty.
template <bool COHERENT, int KEYS>
__device__ __forceinline__ void write_plan_row(const SelectArgs& a, int b, int slot, int committed, int n_sel,
                                               int stored_count, SelectShared<KEYS>& sh) {
  const int tid = threadIdx.x;
  int64_t* prow = a.plan + static_cast<int64_t>(b) * a.plan_width;
  const int64_t cap = min(static_cast<int64_t>(a.plan_width - 5), a.ids_stride);
  const int count = n_sel >= 0 ? n_sel : static_cast<int>(min(static_cast<int64_t>(stored_count), cap));
  const int32_t* stored = a.ids + static_cast<int64_t>(slot) * a.ids_stride;
  auto chunk_id = [&](int j) -> int64_t { return n_sel >= 0 ? sh.ids[j] : stored[j]; };

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
      const int64_t prefix_tokens = block_sum(static_cast<int>(part), sh.scratch);
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
    if constexpr (COHERENT) {
      coherent_store(prow + j, v);
    } else {
      prow[j] = v;
    }
  }
  if (tid == 0 && a.working_lens != nullptr) a.working_lens[slot] = static_cast<int32_t>(len);
}

}  // namespace select
}  // namespace ds355
