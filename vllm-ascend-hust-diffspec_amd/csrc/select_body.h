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
  int32_t* gen;  // [num_slots] selection generation, +1 with every stored selection; or nullptr
};

// LDS of one selecting workgroup of NT threads.  KEYS = candidates whose
// keys stay in LDS.
template <int KEYS, int NT = kThreads>
struct SelectShared {
  alignas(16) uint32_t keys[KEYS + 4];  // + 4: a 4-key read at the end stays inside
  int hist[4][256];  // one histogram per radix pass
  int res[4][3];     // per pass: the digit holding the cut, keys above it, keys in it
  uint32_t range[2][NT / 64];  // per wave: smallest and largest candidate key
  int ids[kMaxSel];
  int scratch[4];
  int wcount[2 * NT / 64];  // per-wave counts of the compaction
  int digit, above, eq;
};

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN: largest
  if ((u & 0x7fffffffu) == 0u) u = 0u;                      // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
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

typedef uint32_t U4 __attribute__((ext_vector_type(4)));

// Top K - 1 of the N candidates (chunks 0..N-1) plus the newest chunk N,
// ascending, into sh.ids[0..K).  key4_at(q) returns the keys of candidates
// 4q .. 4q + 3 (values past N are ignored).  kmin / kmax: bounds of the
// candidate keys this thread has seen (any bounds are correct; the full
// range 0 .. ~0 when unknown).  Starts and ends on a barrier-separated LDS
// state; requires N + 1 > K.
//   - The block's smallest and largest key fix the leading bits every
//     candidate shares; MSB radix passes of up to 8 bits (LDS histogram,
//     wave 0 scans the bins) then start below them, so the first pass
//     spreads keys of a narrow range over many bins instead of piling
//     them into one or two (LDS atomics on one bin serialise).  They find
//     T, the (K-1)-th largest key.  A thread reads 4 keys at a time.  A
//     pass whose bin holding the (K-1)-th key is taken whole ends the
//     search: T is then that bin's prefix with the low bits zero, every key
//     of the bin is > T or == T, and all ties are taken, so the selected
//     set is the one the remaining passes would have found.
//   - Compaction: wave w owns the contiguous candidates
//     [w * span, (w + 1) * span), 256 at a time, lane l holding candidates
//     4l .. 4l + 3 of each 256.  A first sweep counts keys > T and ties
//     (== T) with ballots; one barrier shares the four waves' counts, which
//     fixes each wave's first output slot and how many ties it takes (ties
//     go to the lowest indices); a second sweep writes the ids in order.
template <int KEYS, int NT, typename Key4At>
__device__ __forceinline__ void select_top(SelectShared<KEYS, NT>& sh, int N, int K, Key4At key4_at,
                                           uint32_t kmin = 0u, uint32_t kmax = ~0u) {
  const int tid = threadIdx.x;
  int need = K - 1;
  uint32_t prefix = 0u, pmask = 0u;
  bool take_all_ties = true;
  if (need > 0) {
    // The bounds and the four passes' histograms share one barrier; a pass
    // then takes two: one after its histogram, one after wave 0 has found
    // the digit (lane l scans digits 255 - 4l .. 252 - 4l, the wave's
    // inclusive scan gives each lane the count of keys in higher digits).
    kmin = wave_pick<false>(kmin);
    kmax = wave_pick<true>(kmax);
    if ((tid & 63) == 0) {
      sh.range[0][tid >> 6] = kmin;
      sh.range[1][tid >> 6] = kmax;
    }
    for (int i = tid; i < 4 * 256; i += NT) sh.hist[i >> 8][i & 255] = 0;
    lds_barrier();
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      kmin = min(kmin, sh.range[0][w]);
      kmax = max(kmax, sh.range[1][w]);
    }
    // Bits above `top` are the same in every candidate.
    int top = kmin == kmax ? 0 : 32 - __clz(static_cast<int>(kmin ^ kmax));
    if (top < 32) {
      pmask = ~0u << top;
      prefix = kmax & pmask;
    }
    if (top == 0) take_all_ties = need == N;  // every candidate equals T = kmax
    for (int pass = 0; top > 0; ++pass) {
      const int shift = max(top - 8, 0);
      const uint32_t width_mask = (1u << (top - shift)) - 1u;
      int* hist = sh.hist[pass];
      for (int q = tid; 4 * q < N; q += NT) {
        const U4 k4 = key4_at(q);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (4 * q + j < N && (k4[j] & pmask) == prefix) atomicAdd(&hist[(k4[j] >> shift) & width_mask], 1);
        }
      }
      lds_barrier();
      if (tid < 64) {
        int c[4], sum = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c[e] = hist[255 - 4 * tid - e];
          sum += c[e];
        }
        int before = wave_inclusive_scan(sum) - sum;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (before < need && need <= before + c[e]) {
            sh.res[pass][0] = 255 - 4 * tid - e;
            sh.res[pass][1] = before;
            sh.res[pass][2] = c[e];
          }
          before += c[e];
        }
      }
      lds_barrier();
      prefix |= static_cast<uint32_t>(sh.res[pass][0]) << shift;
      pmask |= width_mask << shift;
      need -= sh.res[pass][1];
      take_all_ties = need == sh.res[pass][2];  // the last pass decides; an earlier one may end the search
      if (take_all_ties) break;  // workgroup-uniform: every thread read the same counts
      top = shift;
    }
  }
  // need = ties (key == T) still to take, lowest indices first.
  const uint32_t T = prefix;
  if (K - 1 > 0) {
    constexpr int kW = NT / 64;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int span = ((N + kW - 1) / kW + 255) / 256 * 256;
    const int lo = min(N, wave * span);
    const int hi = min(N, lo + span);
    int gt = 0, eq = 0;  // this lane's keys > T and == T
    for (int b = lo; b < hi; b += 256) {
      const U4 k4 = key4_at((b >> 2) + lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = b + 4 * lane + j < hi;
        gt += (in && k4[j] > T) ? 1 : 0;
        eq += (in && k4[j] == T) ? 1 : 0;
      }
    }
    gt = wave_total(gt);
    eq = wave_total(eq);
    if (lane == 0) {
      sh.wcount[wave] = gt;
      sh.wcount[kW + wave] = eq;
    }
    lds_barrier();
    int out = 0, eq_before = 0, take_eq = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const int w_eq = sh.wcount[kW + w];
      const int w_take = take_all_ties ? w_eq : max(0, min(w_eq, need - eq_before));
      if (w < wave) out += sh.wcount[w] + w_take;
      if (w == wave) take_eq = w_take;
      eq_before += w_eq;
    }
    // Second sweep, 256 candidates at a time: a wave scan of the lanes' tie
    // counts ranks each tie (lowest index first), a scan of the lanes'
    // selected counts gives each selected id its output slot.
    int taken = 0;  // ties of this wave's earlier candidates
    for (int b = lo; b < hi; b += 256) {
      const U4 k4 = key4_at((b >> 2) + lane);
      bool is_eq[4], sel[4];
      int n_eq = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = b + 4 * lane + j < hi;
        is_eq[j] = in && k4[j] == T;
        n_eq += is_eq[j] ? 1 : 0;
      }
      const int eq_incl = wave_inclusive_scan(n_eq);
      int tie_rank = taken + eq_incl - n_eq;
      int n_sel = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = b + 4 * lane + j < hi;
        sel[j] = in && (k4[j] > T || (is_eq[j] && tie_rank < take_eq));
        tie_rank += is_eq[j] ? 1 : 0;
        n_sel += sel[j] ? 1 : 0;
      }
      const int sel_incl = wave_inclusive_scan(n_sel);
      int pos = out + sel_incl - n_sel;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (sel[j]) {
          if (pos < kMaxSel) sh.ids[pos] = b + 4 * lane + j;
          ++pos;
        }
      }
      out += __builtin_amdgcn_readlane(sel_incl, 63);
      taken += __builtin_amdgcn_readlane(eq_incl, 63);
    }
  }
  if (tid == 0) sh.ids[K - 1] = N;
}

// Plan row of batch row b for a valid slot with `count` chunk ids
// (count < 0: no selection), id j read by chunk_id(j).  Writes plan[b] and
// working_lens[slot]; with a tagged copy, also stores column j as
// (tag << 32) | value in tagged[j] with a device-scope store (plan values
// are below 2^31).  No barriers.
template <int NT, typename ChunkId>
__device__ __forceinline__ void plan_row_from(const SelectArgs& a, int b, int slot, int committed, int count,
                                              ChunkId chunk_id, uint64_t* tagged, uint32_t tag) {
  const int tid = threadIdx.x;
  int64_t* prow = a.plan + static_cast<int64_t>(b) * a.plan_width;
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
      // Every wave sums all terms itself (no barrier): int, each term <=
      // chunk, the total <= count * chunk.
      int part = 0;
      for (int j = tid & 63; j < count; j += 64) {
        const int64_t t = prefix_end - chunk_id(j) * a.chunk;
        part += static_cast<int>(t <= 0 ? 0 : (t < a.chunk ? t : a.chunk));
      }
      const int64_t prefix_tokens = wave_sum_int(part);
      prefix_len = min(prefix_tokens, hb - tail_len);
      drop = prefix_tokens - prefix_len;
      len = prefix_len + tail_len;
    }
  }
  for (int j = tid; j < a.plan_width; j += NT) {
    int64_t v;
    if (j == 0) v = slot;
    else if (j == 1) v = len;
    else if (j == 2) v = tail_start;
    else if (j == 3) v = prefix_len;
    else if (j == 4) v = drop;
    else v = (j - 5) < ncols ? chunk_id(j - 5) : 0;
    prow[j] = v;
    if (tagged != nullptr) {
      coherent_store(tagged + j, (static_cast<uint64_t>(tag) << 32) | static_cast<uint32_t>(v));
    }
  }
  if (tid == 0 && a.working_lens != nullptr) a.working_lens[slot] = static_cast<int32_t>(len);
}

// Plan row of batch row b for a valid slot, from the selection just made
// (n_sel >= 0, ids in sh.ids) or the slot's stored one (n_sel < 0,
// stored_count entries).  The two sources get a loop each: ids read
// through a pointer that may be LDS or global memory compile to flat loads,
// and each of those waited for every store in flight (the selection's own
// ids and scores), a memory round trip per read.
template <int KEYS, int NT>
__device__ __forceinline__ void write_plan_row(const SelectArgs& a, int b, int slot, int committed, int n_sel,
                                               int stored_count, SelectShared<KEYS, NT>& sh,
                                               uint64_t* tagged = nullptr, uint32_t tag = 0) {
  if (n_sel >= 0) {  // workgroup-uniform
    plan_row_from<NT>(a, b, slot, committed, n_sel, [&](int j) -> int64_t { return sh.ids[j]; }, tagged, tag);
  } else {
    const int64_t cap = min(static_cast<int64_t>(a.plan_width - 5), a.ids_stride);
    const int count = static_cast<int>(min(static_cast<int64_t>(stored_count), cap));
    const int32_t* stored = a.ids + static_cast<int64_t>(slot) * a.ids_stride;
    plan_row_from<NT>(a, b, slot, committed, count, [&](int j) -> int64_t { return stored[j]; }, tagged, tag);
  }
}

}  // namespace select
}  // namespace ds355
