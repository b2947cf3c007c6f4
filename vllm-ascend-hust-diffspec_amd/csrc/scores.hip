// Paged chunk scores: one streaming pass over the scored keys.
//
// Counterpart of diffspec/kernels.py:11-150.  The reference launches one
// program per (row, chunk, query head), so every key row is fetched once per
// query head of its GQA group.  Here a workgroup owns one (row, chunk) unit
// across all heads: each key row is loaded once, straight from HBM into the
// B operand of v_mfma_f32_16x16x32_{bf16,f16} (16 tokens x 32 dims per
// instruction, 16 bytes per lane), and multiplied by all query heads of its
// KV head at once (A operand: up to 16 heads x 32 dims, kept in registers).
// The 16x16 fp32 logits come back 4 per lane (rows = heads, column =
// token), are turned into exp(scale*logit - lse) in registers, summed in the
// lane, then across the wave with shuffles and across the 4 waves through
// LDS.  The head mean (kernels.py:150) is fused: out = sum / (Hq * n_valid).
//
// Units (row, chunk) of a ragged batch are numbered by an exclusive prefix
// sum over per-row chunk counts that each workgroup builds in LDS; the grid
// is persistent over that list.
#include "rowdesc.h"

namespace ds355 {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunkForMax = 2048;  // LDS per-token maxima (head_reduce=max)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct alignas(16) Raw16 {
  uint32_t w[4];
};

struct ScoreArgs {
  const uint16_t* q;
  int64_t q_stride;
  const uint16_t* k;
  int64_t k_block_stride, k_token_stride, k_head_stride;
  const float* lse;
  int64_t lse_row_stride, lse_head_stride;
  const int32_t* bt;
  int64_t bt_stride;
  RowSource src;
  int batch, Hq, Hkv, D, block_size, chunk, max_chunks;
  float scale;
  float* out;
  int64_t out_stride;
  int write_tail;
};

template <int DT>
__device__ __forceinline__ f32x4_t mfma16x16x32(const Raw16& a, const Raw16& b, f32x4_t c) {
  if constexpr (DT == DS_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
}

__device__ __forceinline__ int row_units(const ScoreArgs& a, int b) {
  const RowDesc d = row_desc(a.src, b);
  return d.active ? (d.len + a.chunk - 1) / a.chunk : 0;
}

// STEPS = head_dim / 32 (MFMA k-steps per key row).  HMAX selects the
// per-token max over heads instead of the head mean.
template <int DT, int STEPS, bool HMAX>
__global__ __launch_bounds__(kThreads) void chunk_score_kernel(ScoreArgs a) {
  constexpr int kBatch = STEPS >= 16 ? 1 : 16 / STEPS;  // items per load batch (64 VGPRs of keys)
  __shared__ int s_prefix[kMaxRows + 1];
  __shared__ int s_scratch[4];
  __shared__ float s_red[2][4];
  __shared__ unsigned s_tokmax[HMAX ? kMaxChunkForMax : 1];

  if (HMAX) {
    for (int t = threadIdx.x; t < kMaxChunkForMax; t += kThreads) s_tokmax[t] = 0u;
  }
  build_row_prefix(a.batch, s_prefix, s_scratch, [&](int b) { return row_units(a, b); });
  const int total = s_prefix[a.batch];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;   // A row (query head in group) / B column (token in group)
  const int kgrp = lane >> 4;  // which 8-element k slice of the 32-wide step
  const int G = a.Hq / a.Hkv;
  const int NT = (a.chunk + 15) / 16;
  const int items = NT * a.Hkv;                    // (kv head, 16-token group) pairs per unit
  const int per_wave = (items + 3) / 4;
  const int item_begin = wave * per_wave;
  const int item_end = min(items, item_begin + per_wave);
  const float inv_heads = 1.0f / static_cast<float>(a.Hq);

  int parity = 0;
  for (int unit = blockIdx.x; unit < total; unit += gridDim.x, parity ^= 1) {
    const int b = find_row(s_prefix, a.batch, unit);
    const int c = unit - s_prefix[b];
    const RowDesc d = row_desc(a.src, b);
    const int t_begin = c * a.chunk;
    const int n_valid = min(a.chunk, d.len - t_begin);
    const uint16_t* qrow = a.q + d.qrow * a.q_stride;
    const int32_t* bt_row = a.bt + static_cast<int64_t>(b) * a.bt_stride;

    float acc = 0.f;
    int cached_g = -1;
    Raw16 qa[STEPS];
    float lse4[4];

    for (int i0 = item_begin; i0 < item_end; i0 += kBatch) {
      Raw16 kb[kBatch][STEPS];
      // Load phase: all key vectors of the batch are in flight together.
#pragma unroll
      for (int ib = 0; ib < kBatch; ++ib) {
        const int item = i0 + ib;
        const int g = item / NT;
        const int tg = item - g * NT;
        const int tin = tg * 16 + col;
        const int t = t_begin + tin;
        const bool valid = item < item_end && tin < a.chunk && t < d.len;
        if (valid) {
          const int64_t page = bt_row[t / a.block_size];
          const uint16_t* krow = a.k + page * a.k_block_stride + static_cast<int64_t>(t % a.block_size) * a.k_token_stride +
                                 static_cast<int64_t>(g) * a.k_head_stride + kgrp * 8;
#pragma unroll
          for (int s = 0; s < STEPS; ++s) kb[ib][s] = *reinterpret_cast<const Raw16*>(krow + 32 * s);
        } else {
#pragma unroll
          for (int s = 0; s < STEPS; ++s) kb[ib][s] = Raw16{{0u, 0u, 0u, 0u}};
        }
      }
      // Compute phase.
#pragma unroll
      for (int ib = 0; ib < kBatch; ++ib) {
        const int item = i0 + ib;
        if (item >= item_end) continue;  // wave-uniform
        const int g = item / NT;
        const int tg = item - g * NT;
        if (g != cached_g) {
          cached_g = g;
          const bool head_ok = col < G;
          const uint16_t* qh = qrow + static_cast<int64_t>(g * G + col) * a.D + kgrp * 8;
#pragma unroll
          for (int s = 0; s < STEPS; ++s) {
            qa[s] = head_ok ? *reinterpret_cast<const Raw16*>(qh + 32 * s) : Raw16{{0u, 0u, 0u, 0u}};
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * kgrp + i;
            lse4[i] = m < G ? a.lse[d.qrow * a.lse_row_stride + static_cast<int64_t>(g * G + m) * a.lse_head_stride]
                            : 0.f;
          }
        }
        f32x4_t logit = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < STEPS; ++s) logit = mfma16x16x32<DT>(qa[s], kb[ib][s], logit);
        const int tin = tg * 16 + col;
        const bool tok_ok = tin < a.chunk && t_begin + tin < d.len;
        if (HMAX) {
          float m4 = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * kgrp + i;
            if (m < G && tok_ok) m4 = fmaxf(m4, __expf(logit[i] * a.scale - lse4[i]));
          }
          m4 = fmaxf(m4, __shfl_xor(m4, 16, 64));
          m4 = fmaxf(m4, __shfl_xor(m4, 32, 64));
          if (kgrp == 0 && tok_ok) atomicMax(&s_tokmax[tin], __float_as_uint(m4));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * kgrp + i;
            if (m < G && tok_ok) acc += __expf(logit[i] * a.scale - lse4[i]);
          }
        }
      }
    }

    if (HMAX) {
      __syncthreads();
      for (int t = threadIdx.x; t < a.chunk; t += kThreads) {
        acc += __uint_as_float(s_tokmax[t]);
        s_tokmax[t] = 0u;
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) s_red[parity][wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      const float sum = s_red[parity][0] + s_red[parity][1] + s_red[parity][2] + s_red[parity][3];
      const float denom = static_cast<float>(n_valid > 1 ? n_valid : 1);
      a.out[static_cast<int64_t>(b) * a.out_stride + c] = HMAX ? sum / denom : (sum / denom) * inv_heads;
    }
  }

  if (a.write_tail) {
    // Chunks at or beyond a row's length are 0, as in the reference output.
    const int64_t n = static_cast<int64_t>(a.batch) * a.max_chunks;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
      const int b = static_cast<int>(i / a.max_chunks);
      const int c = static_cast<int>(i - static_cast<int64_t>(b) * a.max_chunks);
      if (c >= s_prefix[b + 1] - s_prefix[b]) a.out[static_cast<int64_t>(b) * a.out_stride + c] = 0.f;
    }
  }
}

template <int DT, bool HMAX>
void launch_steps(hipStream_t stream, const ScoreArgs& a, int grid) {
  switch (a.D / 32) {
    case 1: chunk_score_kernel<DT, 1, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    case 2: chunk_score_kernel<DT, 2, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    case 3: chunk_score_kernel<DT, 3, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    case 4: chunk_score_kernel<DT, 4, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    case 5: chunk_score_kernel<DT, 5, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    case 6: chunk_score_kernel<DT, 6, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    case 7: chunk_score_kernel<DT, 7, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
    default: chunk_score_kernel<DT, 8, HMAX><<<grid, kThreads, 0, stream>>>(a); break;
  }
}

}  // namespace

// Shared by ds_chunk_scores and the fused step.
int launch_chunk_scores(hipStream_t stream, int dtype, const void* query, int64_t q_stride, const void* key_cache,
                        int64_t k_block_stride, int64_t k_token_stride, int64_t k_head_stride, const float* lse,
                        int64_t lse_row_stride, int64_t lse_head_stride, const int32_t* block_table,
                        int64_t bt_stride, const RowSource& src, int batch, int num_q_heads, int num_kv_heads,
                        int head_dim, int block_size, int chunk_size, int max_chunks, float scale, int head_reduce,
                        float* out, int64_t out_stride, int write_tail) {
  DS_REQUIRE(dtype == DS_BF16 || dtype == DS_FP16, "chunk scores support BF16 or FP16 query/key caches");
  DS_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
             "query heads must be divisible by KV heads");
  DS_REQUIRE(chunk_size > 0, "chunk_size must be positive");
  DS_REQUIRE(block_size > 0, "block_size must be positive");
  DS_REQUIRE(batch >= 0 && max_chunks >= 0, "batch and max_chunks must be non-negative");
  DS_REQUIRE(head_reduce == DS_HEAD_MEAN || head_reduce == DS_HEAD_MAX, "head_reduce must be mean or max");
  DS_SUPPORTED(head_dim > 0 && head_dim % 32 == 0 && head_dim <= 256, "head_dim must be a multiple of 32 up to 256 (got %d)",
               head_dim);
  DS_SUPPORTED(num_q_heads / num_kv_heads <= 16, "at most 16 query heads per KV head (got %d)",
               num_q_heads / num_kv_heads);
  DS_SUPPORTED(batch <= kMaxRows, "at most %d rows per launch (got %d)", kMaxRows, batch);
  DS_SUPPORTED(head_reduce == DS_HEAD_MEAN || chunk_size <= kMaxChunkForMax,
               "head_reduce=max supports chunks of at most %d tokens", kMaxChunkForMax);
  DS_REQUIRE(q_stride % 8 == 0 && k_block_stride % 8 == 0 && k_token_stride % 8 == 0 && k_head_stride % 8 == 0,
             "query and key strides must be multiples of 8 elements (16-byte rows)");
  DS_REQUIRE((reinterpret_cast<uintptr_t>(query) & 15u) == 0 && (reinterpret_cast<uintptr_t>(key_cache) & 15u) == 0,
             "query and key cache must be 16-byte aligned");
  if (batch == 0 || max_chunks == 0) return clear_error();
  DS_REQUIRE(query && key_cache && lse && block_table && out, "null tensor pointer");
  DS_REQUIRE(src.seq_lens != nullptr || src.counts != nullptr, "null seq_lens pointer");

  ScoreArgs a{};
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
  a.D = head_dim;
  a.block_size = block_size;
  a.chunk = chunk_size;
  a.max_chunks = max_chunks;
  a.scale = scale;
  a.out = out;
  a.out_stride = out_stride;
  a.write_tail = write_tail;

  const int64_t upper = static_cast<int64_t>(batch) * max_chunks;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 8;
  const int grid = static_cast<int>(upper < cap ? upper : cap);
  const bool hmax = head_reduce == DS_HEAD_MAX;
  if (dtype == DS_BF16) {
    if (hmax) launch_steps<DS_BF16, true>(stream, a, grid); else launch_steps<DS_BF16, false>(stream, a, grid);
  } else {
    if (hmax) launch_steps<DS_FP16, true>(stream, a, grid); else launch_steps<DS_FP16, false>(stream, a, grid);
  }
  return check_launch("ds_chunk_scores");
}

}  // namespace ds355

extern "C" int ds_chunk_scores(ds_stream_t stream, int dtype, const void* query, int64_t q_stride,
                               const void* key_cache, int64_t k_block_stride, int64_t k_token_stride,
                               int64_t k_head_stride, const float* lse, int64_t lse_row_stride,
                               int64_t lse_head_stride, const int32_t* block_table, int64_t bt_stride,
                               const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                               int block_size, int chunk_size, int max_chunks, float scale, int head_reduce,
                               float* out, int64_t out_stride) {
  ds355::RowSource src{};
  src.seq_lens = seq_lens;
  return ds355::launch_chunk_scores(reinterpret_cast<hipStream_t>(stream), dtype, query, q_stride, key_cache,
                                    k_block_stride, k_token_stride, k_head_stride, lse, lse_row_stride,
                                    lse_head_stride, block_table, bt_stride, src, batch, num_q_heads, num_kv_heads,
                                    head_dim, block_size, chunk_size, max_chunks, scale, head_reduce, out,
                                    out_stride, 1);
}
