// Per-row retrieval descriptor shared by the scoring and selection kernels.
#pragma once

#include "ds355_common.h"

namespace ds355 {

// Where a row's scores come from.  Direct mode (seq_lens != nullptr) is the
// reference kernel's contract: row b scores seq_lens[b] tokens with query
// row b.  Retrieval mode derives both from the verifier batch, as
// diffspec/runtime.py:1211-1276 does for linear verification:
//   - rows >= batch_size are graph padding and are never scored;
//   - rows with counts[b] <= 0 committed nothing and are skipped;
//   - the query is the last committed one, q_start + clamp(count-1, 0, qlen-1);
//   - the scored length drops the rejected suffix,
//     target_len - qlen + clamp(count, 1, qlen).
struct RowSource {
  const int32_t* seq_lens;
  const int32_t* counts;
  const int32_t* q_start;
  const int32_t* q_len;
  const int32_t* target_len;
  int batch_size;
  int max_len;  // scored lengths are clamped to the score buffer's capacity
};

struct RowDesc {
  int active;  // the row is scored and selected this step
  int len;     // scored length (>= 0; 0 gives an empty selection)
  int64_t qrow;
};

__device__ __forceinline__ RowDesc row_desc(const RowSource& s, int b) {
  RowDesc d{0, 0, 0};
  if (s.seq_lens != nullptr) {
    d.active = 1;
    d.len = s.seq_lens[b];
    d.qrow = b;
  } else {
    if (b >= s.batch_size) return d;
    const int count = s.counts[b];
    const int qlen = s.q_len[b];
    if (count <= 0 || qlen <= 0) return d;
    const int off = min(max(count - 1, 0), qlen - 1);
    d.qrow = static_cast<int64_t>(s.q_start[b]) + off;
    d.active = 1;
    d.len = s.target_len[b] - qlen + min(max(count, 1), qlen);
  }
  if (d.len > s.max_len) d.len = s.max_len;
  if (d.len < 0) d.len = 0;
  return d;
}

// First raw position the draft's prefill of this step rewrites for row b
// (its first verifier query token), for a history gather that runs before
// that prefill: positions below it are final.
__device__ __forceinline__ int first_rewritten(const RowSource& s, int b) {
  return s.target_len[b] - s.q_len[b];
}

// Committed length (root position + 1) of row b for its plan: given per
// row, or, without that array, the scored length of a row that committed
// tokens this step and 0 for any other row (no history to move yet).
__device__ __forceinline__ int committed_of(const int32_t* committed_lens, const RowSource& s, int b) {
  if (committed_lens != nullptr) return committed_lens[b];
  const RowDesc d = row_desc(s, b);
  return d.active ? d.len : 0;
}

}  // namespace ds355
