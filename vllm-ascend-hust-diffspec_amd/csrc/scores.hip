// Paged chunk scores: one streaming pass over the scored keys.
//
// Counterpart of diffspec/kernels.py:11-150.  The reference launches one
// program per (row, chunk, query head), so every key row is fetched once per
// query head of its GQA group.  Here every key row is loaded once, straight
// from HBM into the B operand of v_mfma_f32_16x16x32_{bf16,f16} (16 tokens x
// 32 dims per instruction, 16 bytes per lane), and multiplied by all query
// heads of its KV head at once (A operand: up to 16 heads x 32 dims).  The
// 16x16 fp32 logits come back 4 per lane (rows = heads, column = token) and
// are turned into exp(scale * logit - lse) in registers.
//
// Work decomposition.  A unit is (row, span of U tokens, KV head), U = the
// chunk size rounded up to 64 tokens when the chunk divides 64 (so a unit
// holds 1..4 whole chunks).  Units are numbered through an exclusive prefix
// sum over per-row unit counts built in LDS, and every wave of the persistent
// grid walks its own strided unit list with no block barrier: the units are
// small and uniform, so the static split leaves a short tail.  Each wave runs
// a three-stage software pipeline over 16-token-group batches: block-table
// lookups (uniform, scalar loads) two batches ahead, key / query / LSE loads
// one batch ahead, MFMA + exp on the current batch.  A unit's per-chunk sums
// are reduced across the wave with shuffles and stored as partials
// [row, chunk, KV head]; the head sum and the 1 / (Hq * n_valid)
// normalisation (kernels.py:80-82, 150) happen where the partials are read:
// in the selection kernel for a retrieval step, or in finalize_kernel for
// the drop-in entry point.  The per-token head max (head_reduce = max) keeps
// all KV heads of a span in one wave and writes final scores directly.
//
// Without a supplied LSE (the reference's chunk_attention_scores with
// softmax_lse=None, diffspec/runtime.py:321-322: the LSE of each query head
// over the row's scored tokens) the same single pass keeps, per lane, a
// running (max, sum of 2^(logit - max)) per chunk and query head, merges the
// 16 token lanes with DPP permutes and stores each chunk's log2 mass
// M = max + log2(sum) as one 64-bit word per query head; lse_finalize_kernel
// then merges a row's chunks into each head's LSE and writes the usual
// per-KV-head partials, the sum over the group's heads of 2^(M - lse), so
// selection and the drop-in finalize read them unchanged.
#include "score_body.h"

namespace ds355 {
namespace {

using namespace score;

// STEPS = head_dim / 32.  KB = 16-token groups per batch.  WGS = workgroups
// per CU the register budget is sized for.  HMAX = per-token head max.
// PAGE = how a 16-token group finds its keys (score_body.h): per-lane
// block-table lookups, one scalar lookup per group (block_size and the unit
// start multiples of 16), or the same with power-of-two block size and KV
// heads.
template <int DT, int STEPS, int KB, int WGS, bool HMAX, int PAGE, bool LSEFREE>
__global__ __launch_bounds__(kThreads, WGS) void chunk_score_kernel(ScoreArgs a) {
  __shared__ int s_prefix[kMaxRows + 1];
  __shared__ int s_len[kMaxRows];
  __shared__ int s_qrow[kMaxRows];
  __shared__ int s_scratch[4];

  const int units_per_span = HMAX ? 1 : a.Hkv;
  for (int r = threadIdx.x; r < a.batch; r += kThreads) {
    const RowDesc d = row_desc(a.src, r);
    s_len[r] = d.active ? d.len : 0;
    s_qrow[r] = static_cast<int>(d.qrow);
  }
  __syncthreads();
  build_row_prefix(a.batch, s_prefix, s_scratch,
                   [&](int r) { return (s_len[r] + a.U - 1) / a.U * units_per_span; });
  const int total = s_prefix[a.batch];
  const int gw = uniform(blockIdx.x * kWaves + (threadIdx.x >> 6));
  score_stream<DT, STEPS, KB, HMAX, PAGE, false, LSEFREE>(a, s_prefix, s_len, s_qrow, total, gw,
                                                                  gridDim.x * kWaves, 0u);

  if (a.write_tail) {
    // Head max writes final scores; chunks at or beyond a row's length are 0.
    const int64_t n = static_cast<int64_t>(a.batch) * a.max_chunks;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
      const int b = static_cast<int>(i / a.max_chunks);
      const int c = static_cast<int>(i - static_cast<int64_t>(b) * a.max_chunks);
      if (c >= (s_len[b] + a.chunk - 1) / a.chunk) a.out[static_cast<int64_t>(b) * a.out_stride + c] = 0.f;
    }
  }
}

// Drop-in output: out[b, c] = sum_g partial[b, c, g] / n_valid / Hq, 0 past the row.
__global__ __launch_bounds__(kThreads) void finalize_kernel(const float* __restrict__ partial,
                                                            const int32_t* __restrict__ seq_lens, int batch,
                                                            int max_chunks, int hkv, int hq, int chunk, int max_len,
                                                            float* __restrict__ out, int64_t out_stride) {
  const int64_t n = static_cast<int64_t>(batch) * max_chunks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int b = static_cast<int>(i / max_chunks);
    const int c = static_cast<int>(i - static_cast<int64_t>(b) * max_chunks);
    const int len = min(max(seq_lens[b], 0), max_len);
    float v = 0.f;
    if (c * chunk < len) {
      float s = 0.f;
      for (int g = 0; g < hkv; ++g) s += partial[i * hkv + g];
      const int n_valid = min(chunk, len - c * chunk);
      v = (s / static_cast<float>(n_valid)) / static_cast<float>(hq);
    }
    out[static_cast<int64_t>(b) * out_stride + c] = v;
  }
}

// Scores without a supplied LSE, after the pass: lse_finalize_kernel, one
// workgroup per (row, KV head, slice of finalize_slice(max_chunks) chunks:
// 128, more when a row would need more than kMaxSlices slices).
//   - The group's query heads merge all of the row's mass words into their
//     LSEs (lse_layout / lse_finish, the merge the single launch's selectors
//     run too).  The slice-0 workgroup writes the LSEs (natural log) to
//     lse_out.
//   - Then the KV head's partial of every chunk of the slice, the sum over
//     the group's heads of 2^(M - lse2), which selection and the drop-in
//     finalize read as with a supplied LSE.  The exponent uses the LSE as
//     written (natural log, fp32) times log2(e).
// Every slice of a row repeats the merge (its words come from L2 after the
// first), which costs less than a second launch waiting on the first; the
// cap on slices bounds the repeats at kMaxSlices reads of a row's words.
// `wide` (16-byte aligned words): two heads per thread and 16-byte reads.
constexpr int kFinalizeSlice = 128;  // chunks per workgroup, at least
constexpr int kMaxSlices = 8;        // workgroups per (row, KV head), at most
__host__ __device__ inline int finalize_slice(int max_chunks) {
  const int even = (max_chunks + kMaxSlices - 1) / kMaxSlices;
  return even > kFinalizeSlice ? even : kFinalizeSlice;
}
__global__ __launch_bounds__(kThreads) void lse_finalize_kernel(const uint64_t* __restrict__ mw, RowSource src,
                                                                int max_chunks, int hq, int hkv, int chunk,
                                                                float* __restrict__ lse_out, int64_t lse_stride,
                                                                float* __restrict__ partial, int wide) {
  __shared__ float s_m[2][kThreads], s_z[2][kThreads];
  __shared__ float s_lse2[kMaxGroup];
  const int slice = finalize_slice(max_chunks);
  const int slices = (max_chunks + slice - 1) / slice;
  const int s = blockIdx.x % slices;
  const int g = (blockIdx.x / slices) % hkv;
  const int b = blockIdx.x / slices / hkv;
  const RowDesc d = row_desc(src, b);
  const int len = d.active ? d.len : 0;
  const int chunks = (len + chunk - 1) / chunk;
  const int c_begin = s * slice;
  if (c_begin >= chunks) return;  // workgroup-uniform (also rows with nothing scored)
  const int c_end = min(chunks, c_begin + slice);
  const int G = hq / hkv;
  const int t = threadIdx.x;
  // Words [row, chunk, Hq]: head h of this group's chunk c at words[c * hq + h].
  const uint64_t* words = mw + static_cast<int64_t>(b) * max_chunks * hq + g * G;

  const LseLayout l = lse_layout(G, wide, t);
  LseAcc acc;
  if (l.ph < l.P) {
    const uint64_t* p = words + l.hp * l.ph;
    for (int c0 = l.j; c0 < chunks; c0 += kLseLoads * l.tpp) {
      if (l.hp == 2) {  // workgroup-uniform
        WordPair v[kLseLoads];
#pragma unroll
        for (int u = 0; u < kLseLoads; ++u) {
          const int c = c0 + u * l.tpp;
          v[u] = c < chunks ? *reinterpret_cast<const WordPair*>(p + static_cast<int64_t>(c) * hq)
                            : WordPair{kNoMassWord, kNoMassWord};
        }
#pragma unroll
        for (int u = 0; u < kLseLoads; ++u) acc.add(v[u].a, v[u].b, 2);
      } else {
        uint64_t v[kLseLoads];
#pragma unroll
        for (int u = 0; u < kLseLoads; ++u) {
          const int c = c0 + u * l.tpp;
          v[u] = c < chunks ? p[static_cast<int64_t>(c) * hq] : kNoMassWord;
        }
#pragma unroll
        for (int u = 0; u < kLseLoads; ++u) acc.add(v[u], 0u, 1);
      }
    }
  }
  const float lse = lse_finish(l, acc, G, s_m, s_z);
  if (t < G) {
    if (s == 0) lse_out[static_cast<int64_t>(b) * lse_stride + g * G + t] = lse;
    s_lse2[t] = lse_base2(lse);
  }
  __syncthreads();

  for (int c = c_begin + t; c < c_end; c += kThreads) {
    uint64_t v[kMaxGroup];
    const uint64_t* at = words + static_cast<int64_t>(c) * hq;
    if (l.hp == 2) {
#pragma unroll
      for (int h = 0; h < kMaxGroup; h += 2) {
        const WordPair w = h < G ? *reinterpret_cast<const WordPair*>(at + h) : WordPair{kNoMassWord, kNoMassWord};
        v[h] = w.a;
        v[h + 1] = w.b;
      }
    } else {
#pragma unroll
      for (int h = 0; h < kMaxGroup; ++h) v[h] = h < G ? at[h] : kNoMassWord;
    }
    float sum = 0.f;
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) sum = h < G ? add_share(sum, mass_of(v[h]), s_lse2[h]) : sum;
    partial[(static_cast<int64_t>(b) * max_chunks + c) * hkv + g] = sum;
  }
}

template <int DT, int STEPS, bool HMAX, bool LSEFREE>
void launch_kb(hipStream_t stream, const ScoreArgs& a, int64_t upper_blocks, int page_mode) {
  // Batch shape: about 4 KB of keys per wave and batch at three workgroups
  // per CU.  At head_dim 128 one 16-token group (4 KB) beat two (8 KB) by
  // 1.3 us on 16 rows of 4k-40k tokens and 0.4-0.7 us on 16 x 40k and
  // 4 x 128k, and both beat 16 KB batches at two workgroups per CU (5.4 vs
  // 5.1 TB/s on 16 x 40k); three workgroups also beat four.  At head_dim 64
  // two groups (4 KB) beat four (8 KB) by 2.1-2.9 us and one (2 KB) by
  // 1.4-3.7 us on the same rows.  The single launch uses the same shape
  // (fused.hip), which keeps the two paths' results identical without a
  // supplied LSE.  Wider heads read one group per batch (8 KB at head_dim
  // 256: 1-2 us faster than two groups on 16 rows of 4k-40k tokens) at two
  // workgroups per CU (three measured slower); the head max keeps its wider
  // batches at two workgroups per CU.
  constexpr bool narrow = !HMAX && STEPS <= 4;
  constexpr int KB = narrow ? (STEPS <= 2 ? 2 : 1)
                            : (HMAX ? ((16 / STEPS) >= 4 ? 4 : ((16 / STEPS) >= 2 ? 2 : 1)) : 1);
  constexpr int WGS = narrow ? 3 : 2;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * WGS;
  const int grid = static_cast<int>(std::max<int64_t>(1, std::min(upper_blocks, cap)));
  if (page_mode == PAGE_POW2) {
    chunk_score_kernel<DT, STEPS, KB, WGS, HMAX, PAGE_POW2, LSEFREE><<<grid, kThreads, 0, stream>>>(a);
  } else if (page_mode == PAGE_UNIFORM) {
    chunk_score_kernel<DT, STEPS, KB, WGS, HMAX, PAGE_UNIFORM, LSEFREE><<<grid, kThreads, 0, stream>>>(a);
  } else {
    chunk_score_kernel<DT, STEPS, KB, WGS, HMAX, PAGE_LANE, LSEFREE><<<grid, kThreads, 0, stream>>>(a);
  }
}

template <int DT, bool HMAX, bool LSEFREE>
void launch_steps(hipStream_t stream, const ScoreArgs& a, int64_t grid, int page_mode) {
  switch (a.D / 32) {
    case 1: launch_kb<DT, 1, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    case 2: launch_kb<DT, 2, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    case 3: launch_kb<DT, 3, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    case 4: launch_kb<DT, 4, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    case 5: launch_kb<DT, 5, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    case 6: launch_kb<DT, 6, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    case 7: launch_kb<DT, 7, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
    default: launch_kb<DT, 8, HMAX, LSEFREE>(stream, a, grid, page_mode); break;
  }
}

}  // namespace

// Shared by ds_chunk_scores and the fused step.  With head_reduce = mean the
// kernel writes per-KV-head partials ([batch, max_chunks, Hkv] in `partial`);
// with max it writes final scores to `out` (and zero tails if write_tail).
int make_score_args(ScoreArgs& a, int64_t& upper_units, int& page_mode, int dtype, const void* query,
                    int64_t q_stride, const void* key_cache, int64_t k_block_stride, int64_t k_token_stride,
                    int64_t k_head_stride, const float* lse, int64_t lse_row_stride, int64_t lse_head_stride,
                    const int32_t* block_table, int64_t bt_stride, const RowSource& src, int batch, int num_q_heads,
                    int num_kv_heads, int head_dim, int block_size, int chunk_size, int max_chunks, float scale,
                    int head_reduce, float* partial, float* out, int64_t out_stride, int write_tail,
                    size_t partial_bytes, uint64_t* mw) {
  upper_units = 0;
  page_mode = PAGE_LANE;
  DS_REQUIRE(dtype == DS_BF16 || dtype == DS_FP16, "chunk scores support BF16 or FP16 query/key caches");
  DS_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
             "query heads must be divisible by KV heads");
  DS_REQUIRE(chunk_size > 0, "chunk_size must be positive");
  DS_REQUIRE(block_size > 0, "block_size must be positive");
  DS_REQUIRE(batch >= 0 && max_chunks >= 0, "batch and max_chunks must be non-negative");
  DS_REQUIRE(head_reduce == DS_HEAD_MEAN || head_reduce == DS_HEAD_MAX, "head_reduce must be mean or max");
  DS_SUPPORTED(head_dim > 0 && head_dim % 32 == 0 && head_dim <= 256,
               "head_dim must be a multiple of 32 up to 256 (got %d)", head_dim);
  DS_SUPPORTED(num_q_heads / num_kv_heads <= kMaxGroup, "at most %d query heads per KV head (got %d)", kMaxGroup,
               num_q_heads / num_kv_heads);
  DS_SUPPORTED(batch <= kMaxRows, "at most %d rows per launch (got %d)", kMaxRows, batch);
  DS_REQUIRE(q_stride % 8 == 0 && k_block_stride % 8 == 0 && k_token_stride % 8 == 0 && k_head_stride % 8 == 0,
             "query and key strides must be multiples of 8 elements (16-byte rows)");
  DS_REQUIRE((reinterpret_cast<uintptr_t>(query) & 15u) == 0 && (reinterpret_cast<uintptr_t>(key_cache) & 15u) == 0,
             "query and key cache must be 16-byte aligned");
  // A query group's and an LSE group's loads use 32-bit byte offsets.
  DS_SUPPORTED(lse_head_stride >= 0 && lse_head_stride <= (static_cast<int64_t>(INT32_MAX) / 4 - 1) / kMaxGroup,
               "softmax LSE head stride %lld is too large", static_cast<long long>(lse_head_stride));
  const bool hmax = head_reduce == DS_HEAD_MAX;
  // Unit span: whole chunks, at least 64 tokens when the chunk divides 64.
  int cpu = 1;
  if (chunk_size % 16 == 0 && chunk_size < 64 && 64 % chunk_size == 0) cpu = 64 / chunk_size;
  const int U = cpu * chunk_size;
  const int ntu = (U + 15) / 16;
  DS_SUPPORTED(!hmax || ntu <= kMaxNtu, "head_reduce=max supports chunks of at most %d tokens", kMaxNtu * 16);
  if (batch == 0 || max_chunks == 0) return clear_error();
  DS_REQUIRE(query && key_cache && block_table, "null tensor pointer");
  // No LSE: the pass computes it (head mean only); the mass words need mw.
  DS_SUPPORTED(lse || !hmax, "head_reduce=max needs a supplied softmax LSE");
  DS_REQUIRE(lse || (reinterpret_cast<uintptr_t>(mw) & 7u) == 0,
             "the mass words without an LSE (lse_partials / workspace) must be 8-byte aligned");
  DS_REQUIRE(lse || mw,
             "workspace too small: need %zu bytes without an LSE (batch * (max_chunks * (kv_heads + 2 * q_heads) + "
             "q_heads) * 4)",
             static_cast<size_t>(batch) *
                 (max_chunks * (num_kv_heads + 2 * static_cast<size_t>(num_q_heads)) + num_q_heads) * sizeof(float));
  if (!hmax) {
    const size_t need = static_cast<size_t>(batch) * max_chunks * num_kv_heads * sizeof(float);
    DS_REQUIRE(partial != nullptr && partial_bytes >= need,
               "workspace too small: need %zu bytes (batch * max_chunks * kv_heads * 4)", need);
  }
  DS_REQUIRE(!hmax || out != nullptr, "null score output pointer");
  DS_REQUIRE(src.seq_lens != nullptr || src.counts != nullptr, "null seq_lens pointer");

  a = ScoreArgs{};
  a.q = static_cast<const uint16_t*>(query);
  a.q_stride = q_stride;
  a.k = static_cast<const uint16_t*>(key_cache);
  a.k_block_stride = k_block_stride;
  a.k_token_stride = k_token_stride;
  a.k_head_stride = k_head_stride;
  a.lse = lse;
  a.lse_row_stride = lse_row_stride;
  a.lse_head_stride = lse_head_stride;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.src = src;
  a.src.max_len = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(max_chunks) * chunk_size, INT32_MAX));
  a.batch = batch;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.G = num_q_heads / num_kv_heads;
  a.D = head_dim;
  a.block_size = block_size;
  a.chunk = chunk_size;
  a.max_chunks = max_chunks;
  a.U = U;
  a.cpu = cpu;
  a.ntu = ntu;
  auto log2_or_neg = [](int v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
  };
  a.hkv_log2 = log2_or_neg(num_kv_heads);
  a.bs_log2 = log2_or_neg(block_size);
  // cpu > 1 only for chunks of 16 or 32 tokens (powers of two).
  a.ci_shift = cpu > 1 ? log2_or_neg(chunk_size) : 31;
  a.scale = scale;
  a.partial = partial;
  a.mw = lse ? nullptr : mw;
  a.out = out;
  a.out_stride = out_stride;
  a.write_tail = hmax ? write_tail : 0;

  const int64_t spans = (static_cast<int64_t>(max_chunks) * chunk_size + U - 1) / U;
  upper_units = static_cast<int64_t>(batch) * spans * (hmax ? 1 : num_kv_heads);
  // The uniform paths load a 16-token group through a buffer resource with
  // 32-bit byte offsets: 16 key rows must span less than 2 GiB.
  page_mode = PAGE_LANE;
  if (block_size % 16 == 0 && U % 16 == 0 && k_token_stride <= (static_cast<int64_t>(INT32_MAX) / 32)) {
    page_mode = a.bs_log2 >= 0 && a.hkv_log2 >= 0 ? PAGE_POW2 : PAGE_UNIFORM;
  }
  return clear_error();
}

int launch_chunk_scores(hipStream_t stream, int dtype, const void* query, int64_t q_stride, const void* key_cache,
                        int64_t k_block_stride, int64_t k_token_stride, int64_t k_head_stride, const float* lse,
                        int64_t lse_row_stride, int64_t lse_head_stride, const int32_t* block_table,
                        int64_t bt_stride, const RowSource& src, int batch, int num_q_heads, int num_kv_heads,
                        int head_dim, int block_size, int chunk_size, int max_chunks, float scale, int head_reduce,
                        float* partial, float* out, int64_t out_stride, int write_tail, size_t partial_bytes,
                        uint64_t* mw, float* lse_out, int64_t lse_out_stride) {
  ScoreArgs a{};
  int64_t upper_units = 0;
  int page_mode = PAGE_LANE;
  const int rc = make_score_args(a, upper_units, page_mode, dtype, query, q_stride, key_cache, k_block_stride,
                                 k_token_stride, k_head_stride, lse, lse_row_stride, lse_head_stride, block_table,
                                 bt_stride, src, batch, num_q_heads, num_kv_heads, head_dim, block_size, chunk_size,
                                 max_chunks, scale, head_reduce, partial, out, out_stride, write_tail, partial_bytes,
                                 mw);
  if (rc != DS_OK || upper_units == 0) return rc;
  const bool hmax = head_reduce == DS_HEAD_MAX;
  const bool lse_free = lse == nullptr;
  // Everything the LSE kernel needs is checked before the first launch.
  const int64_t partial_grid =
      static_cast<int64_t>(batch) * num_kv_heads *
      ((max_chunks + finalize_slice(max_chunks) - 1) / finalize_slice(max_chunks));
  if (lse_free) {
    DS_REQUIRE(lse_out != nullptr, "null LSE output pointer (the scores without a supplied LSE compute it there)");
    DS_REQUIRE(lse_out_stride >= num_q_heads, "LSE output rows must hold every query head");
    DS_SUPPORTED(partial_grid < (int64_t{1} << 31), "too many (row, KV head, chunk slice) workgroups");
  }
  const int64_t upper_blocks = (upper_units + kWaves - 1) / kWaves;
  if (dtype == DS_BF16) {
    if (hmax) launch_steps<DS_BF16, true, false>(stream, a, upper_blocks, page_mode);
    else if (lse_free) launch_steps<DS_BF16, false, true>(stream, a, upper_blocks, page_mode);
    else launch_steps<DS_BF16, false, false>(stream, a, upper_blocks, page_mode);
  } else {
    if (hmax) launch_steps<DS_FP16, true, false>(stream, a, upper_blocks, page_mode);
    else if (lse_free) launch_steps<DS_FP16, false, true>(stream, a, upper_blocks, page_mode);
    else launch_steps<DS_FP16, false, false>(stream, a, upper_blocks, page_mode);
  }
  int rc2 = check_launch("ds_chunk_scores");
  if (rc2 != DS_OK || !lse_free) return rc2;
  lse_finalize_kernel<<<static_cast<unsigned>(partial_grid), kThreads, 0, stream>>>(
      a.mw, a.src, max_chunks, num_q_heads, num_kv_heads, chunk_size, lse_out, lse_out_stride, partial,
      lse_words_wide(a.mw));
  return check_launch("ds_chunk_scores lse");
}

}  // namespace ds355

extern "C" int ds_chunk_scores(ds_stream_t stream, int dtype, const void* query, int64_t q_stride,
                               const void* key_cache, int64_t k_block_stride, int64_t k_token_stride,
                               int64_t k_head_stride, const float* lse, int64_t lse_row_stride,
                               int64_t lse_head_stride, const int32_t* block_table, int64_t bt_stride,
                               const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                               int block_size, int chunk_size, int max_chunks, float scale, int head_reduce,
                               float* out, int64_t out_stride, float* workspace, size_t workspace_bytes) {
  using namespace ds355;
  RowSource src{};
  src.seq_lens = seq_lens;
  const bool hmax = head_reduce == DS_HEAD_MAX;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Without an LSE the workspace holds the mass words first ([batch,
  // max_chunks, Hq] 64-bit words at the workspace's start), then each row's
  // LSE ([batch, Hq]), then the per-KV-head partials; a workspace too small
  // for all three is reported with the other argument checks.
  uint64_t* mw = nullptr;
  float* lse_rows = nullptr;
  float* partial = workspace;
  size_t partial_bytes = workspace_bytes;
  if (lse == nullptr && !hmax && batch > 0 && max_chunks > 0 && num_q_heads > 0 && num_kv_heads > 0) {
    const size_t pairs = static_cast<size_t>(batch) * max_chunks * num_q_heads * 2;
    const size_t lses = static_cast<size_t>(batch) * num_q_heads;
    const size_t need = (static_cast<size_t>(batch) * max_chunks * num_kv_heads + pairs + lses) * sizeof(float);
    if (workspace != nullptr && workspace_bytes >= need) {
      mw = reinterpret_cast<uint64_t*>(workspace);
      lse_rows = workspace + pairs;
      partial = lse_rows + lses;
      partial_bytes = workspace_bytes - (pairs + lses) * sizeof(float);
    }
  }
  int rc = launch_chunk_scores(s, dtype, query, q_stride, key_cache, k_block_stride, k_token_stride, k_head_stride,
                               lse, lse_row_stride, lse_head_stride, block_table, bt_stride, src, batch, num_q_heads,
                               num_kv_heads, head_dim, block_size, chunk_size, max_chunks, scale, head_reduce,
                               partial, out, out_stride, 1, partial_bytes, mw, lse_rows, num_q_heads);
  if (rc != DS_OK || hmax || batch == 0 || max_chunks == 0) return rc;
  DS_REQUIRE(out != nullptr, "null score output pointer");
  const int64_t n = static_cast<int64_t>(batch) * max_chunks;
  const int grid = static_cast<int>(std::min<int64_t>((n + kThreads - 1) / kThreads, 4096));
  const int max_len = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(max_chunks) * chunk_size, INT32_MAX));
  finalize_kernel<<<grid, kThreads, 0, s>>>(partial, seq_lens, batch, max_chunks, num_kv_heads, num_q_heads,
                                            chunk_size, max_len, out, out_stride);
  return check_launch("ds_chunk_scores finalize");
}
