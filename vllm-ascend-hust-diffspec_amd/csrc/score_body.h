// Streaming pass over the scored keys, shared by chunk_score_kernel and the
// fused retrieval step.  See scores.hip for the algorithm.
#pragma once

#include "rowdesc.h"

namespace ds355 {
namespace score {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxNtu = 8;  // 16-token groups per unit with head_reduce = max (U <= 128)
constexpr int kMaxGroup = 16;  // query heads per KV head (one 16-row MFMA A operand)

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
  int batch, Hq, Hkv, G, D, block_size, chunk, max_chunks;
  int U;    // tokens per unit
  int cpu;  // chunks per unit
  int ntu;  // 16-token groups per unit
  int hkv_log2, bs_log2;  // log2 when a power of two, else -1
  int ci_shift;  // chunk of a unit's token t = t >> ci_shift (31 when a unit is one chunk)
  float scale;
  union {
    float* partial;    // [batch, max_chunks, Hkv] (head mean) — per-KV-head sums
    uint64_t* tagged;  // fused step: the same sums as (tag << 32) | fp32 bits, stored coherently
  };
  float* out;      // [batch, out_stride] final scores (head max; tail zeros)
  int64_t out_stride;
  int write_tail;
  // Without a supplied LSE: per (row, chunk, query head) one 64-bit word
  // [batch, max_chunks, Hq] (a chunk's heads are contiguous).  Its low half
  // is the chunk's mass in log2 units, M = log2(sum_t 2^(scaled logit_t)),
  // as fp32; its high half is 0 (kernel chain) or the launch's tag (single
  // launch, stored coherently: a reader polling the word needs no other
  // signal).  Chain words never carry a tag, since tags are never 0.
  uint64_t* mw;
};

// The mass M of a word (see ScoreArgs::mw) and the tag it carries.
__device__ __forceinline__ float mass_of(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }
__device__ __forceinline__ uint32_t tag_of(uint64_t w) { return static_cast<uint32_t>(w >> 32); }
constexpr uint64_t kNoMassWord = 0xff800000u;  // M = -inf, no tag
struct alignas(16) WordPair {  // two adjacent heads' words, one 16-byte access
  uint64_t a, b;
};

// (m, z) pairs with m in log2 units: the merged pair of two parts of one sum.
// m = -inf marks an empty part (z = 0).
__device__ __forceinline__ void merge_mz(float& m, float& z, float m2, float z2) {
  const float mn = fmaxf(m, m2);
  const float a = m == -INFINITY ? 0.f : z * __builtin_amdgcn_exp2f(m - mn);
  const float b = m2 == -INFINITY ? 0.f : z2 * __builtin_amdgcn_exp2f(m2 - mn);
  m = mn;
  z = a + b;
}

// Add one term 2^x to the pair (m, z), with one exp2: for x <= m the term is
// 2^(x - m) on the current scale, else the sum is rescaled to x.  m starts at
// kNoMax (finite, so x = -inf adds nothing and the first real x takes over);
// lanes that saw no term keep z = 0.
constexpr float kNoMax = -3.0e38f;
__device__ __forceinline__ void add_term(float& m, float& z, float x) {
  const float d = x - m;
  const float e = __builtin_amdgcn_exp2f(-fabsf(d));
  z = d <= 0.f ? z + e : fmaf(z, e, 1.f);
  m = fmaxf(m, x);
}

// Merge the (m, z) pairs of the 16 lanes of each 16-lane row with DPP lane
// permutes (quad xor 1, quad xor 2, half-row mirror, row mirror): the row's
// max first, then every z rescaled to it once and summed; every lane of the
// row ends with the row's pair.  A lane that saw no term has z = 0 and adds
// nothing, whatever its m.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ void merge_mz_row16(float& m, float& z) {
  float mx = fmaxf(m, dpp_row<0xB1>(m));
  mx = fmaxf(mx, dpp_row<0x4E>(mx));
  mx = fmaxf(mx, dpp_row<0x141>(mx));
  mx = fmaxf(mx, dpp_row<0x140>(mx));
  float t = z > 0.f ? z * __builtin_amdgcn_exp2f(m - mx) : 0.f;
  t += dpp_row<0xB1>(t);
  t += dpp_row<0x4E>(t);
  t += dpp_row<0x141>(t);
  t += dpp_row<0x140>(t);
  m = mx;
  z = t;
}

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

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Raw buffer loads from a wave-uniform base (a resource in scalar registers)
// at loop-invariant per-lane byte offsets: a batch's loads need no address
// arithmetic in vector registers (which also made the compiler wait for
// loads in flight before reusing the registers).
typedef __amdgpu_buffer_rsrc_t SRsrc;
constexpr int kCoherentStorePolicy = 16;  // sc1: the cache policy of device-scope relaxed atomic stores
__device__ __forceinline__ SRsrc srsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ Raw16 bload16(SRsrc r, int voff) {
  return __builtin_bit_cast(Raw16, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ float bload4(SRsrc r, int voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}



// Where a batch sits in the wave's stream.  All fields are wave-uniform and
// 32-bit (the element offsets they imply are worked out where they are used,
// so two batches and a unit in flight fit the scalar registers).
struct BatchCtx {
  int valid;
  int b;     // row
  int qrow;  // query / LSE row
  int t0;    // first token of the unit
  int len;   // row's scored length
  int g;     // KV head
  int tg0;   // first 16-token group of the batch within the unit
  int last;  // last batch of the unit
  int c0;    // first chunk of the unit
  int chunks_row;  // chunks of the row, ceil(len / chunk)
};

// How a 16-token group finds its keys.  PAGE_LANE: per-lane block-table
// lookups (blocks not 16-token aligned).  PAGE_UNIFORM: one scalar lookup per
// group.  PAGE_POW2: the same with power-of-two block size and KV-head count,
// so the per-unit and per-group index maths are shifts and masks.
constexpr int PAGE_LANE = 0;
constexpr int PAGE_UNIFORM = 1;
constexpr int PAGE_POW2 = 2;

template <int KB, int STEPS>
struct Batch {
  Raw16 k[KB][STEPS];
  Raw16 q[STEPS];
  float lse[4];
  BatchCtx c;
  int fresh;  // q and lse were loaded for this batch (else: the same as the batch before)
};

// LSEFREE: merge a chunk's running pairs (one per token group slot of a
// batch, then the 16 token lanes), store each real head's mass word at
// mw[row, chunk, head] and reset for the next chunk.  A unit's G words are
// one contiguous run, and the waves of a workgroup walk consecutive units
// (the KV heads of one span, with 4 KV heads), so a chunk's Hq words are
// written whole by one CU.  Scattered 8-byte pieces of lines shared with
// other XCDs (the [row, head, chunk] order) cost 4 us of a 61 us pass on
// 16 x 40k-token rows.
template <int KB, bool TAGGED>
__device__ __forceinline__ void flush_mass(const ScoreArgs& a, const BatchCtx& c, int cc, float (&m)[KB][4],
                                           float (&z)[KB][4], int kgrp, int col, uint32_t tag) {
  const int ch = c.c0 + cc;
  const int chunks_row = (c.len + a.chunk - 1) / a.chunk;
  float mass[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float mt = m[0][e], zt = z[0][e];
#pragma unroll
    for (int i = 1; i < KB; ++i) merge_mz(mt, zt, m[i][e], z[i][e]);
    merge_mz_row16(mt, zt);
    mass[e] = zt > 0.f ? mt + __log2f(zt) : -INFINITY;
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      m[i][e] = kNoMax;
      z[i][e] = 0.f;
    }
  }
  // Lane (kgrp, col 0) holds heads 4 kgrp .. 4 kgrp + 3 of the group: two
  // adjacent heads' words go out as one 16-byte store where both exist and
  // the address allows (half the store instructions of 8-byte words; each
  // 8-byte word is still written whole).
  if (col == 0 && ch < chunks_row) {
    const int64_t row_words = static_cast<int64_t>(c.b) * a.max_chunks * a.Hq;
    const int at0 = ch * a.Hq + c.g * a.G + 4 * kgrp;  // within the row
    const uint64_t tg = static_cast<uint64_t>(TAGGED ? tag : 0u) << 32;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int h = 4 * kgrp + 2 * p;
      if (h < a.G) {
        const uint64_t w0 = tg | __float_as_uint(mass[2 * p]);
        const uint64_t w1 = tg | __float_as_uint(mass[2 * p + 1]);
        uint64_t* dst = a.mw + row_words + at0 + 2 * p;
        const bool pair = h + 1 < a.G && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
        if constexpr (TAGGED) {
          if (pair) {
            const SRsrc r = srsrc(a.mw + row_words, a.max_chunks * a.Hq * static_cast<int>(sizeof(uint64_t)));
            const uint32_t v[4] = {static_cast<uint32_t>(w0), static_cast<uint32_t>(w0 >> 32),
                                   static_cast<uint32_t>(w1), static_cast<uint32_t>(w1 >> 32)};
            typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
            __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{v[0], v[1], v[2], v[3]}, r,
                                                   (at0 + 2 * p) * static_cast<int>(sizeof(uint64_t)), 0,
                                                   kCoherentStorePolicy);
          } else {
            __hip_atomic_store(dst, w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (h + 1 < a.G) __hip_atomic_store(dst + 1, w1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        } else {
          if (pair) {
            *reinterpret_cast<WordPair*>(dst) = WordPair{w0, w1};
          } else {
            dst[0] = w0;
            if (h + 1 < a.G) dst[1] = w1;
          }
        }
      }
    }
  }
}

// One wave's walk over its strided unit list: units gw, gw + tw, ... of the
// numbering in s_prefix (rows' unit counts, exclusive prefix) with s_len /
// s_qrow the rows' scored lengths and query rows.  Head mean stores
// per-KV-head chunk sums (partial, or tagged with `tag` when TAGGED); head
// max stores final chunk scores.  LSEFREE (head mean only): no LSE is read;
// each chunk's mass word per query head goes to a.mw instead (tagged when
// TAGGED).
template <int DT, int STEPS, int KB, bool HMAX, int PAGE, bool TAGGED, bool LSEFREE = false>
__device__ __forceinline__ void score_stream(const ScoreArgs& a, const int* s_prefix, const int* s_len,
                                             const int* s_qrow, int total, int gw, int tw, uint32_t tag) {
  constexpr bool UNIFORM_PAGE = PAGE != PAGE_LANE;
  constexpr bool POW2 = PAGE == PAGE_POW2;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;   // A row (query head in group) / B column (token in group)
  const int kgrp = lane >> 4;  // 8-element k slice of the 32-wide MFMA step
  const int bph = (a.ntu + KB - 1) / KB;     // batches per KV head of a unit
  const int bpu = bph * (HMAX ? a.Hkv : 1);  // batches per unit

  // The wave's cursor: unit ordinal uk (unit gw + uk * tw), batch uj within
  // it, and for the head max the head hj and group batch tj within the
  // span.  Everything a unit's batches share is worked out once, when the
  // unit starts; a batch only moves its group offset.  next_ctx() hands out
  // the batches in order, two ahead of the one being computed.  (Integer
  // division per batch, and both arms of shift-or-divide selects, were most
  // of the pass's scalar instructions: about 430 per 8 KB batch.)
  int uk = 0, uj = 0, hj = 0, tj = 0;
  int row_hint = 0;
  BatchCtx u{};  // the current unit
  auto next_ctx = [&]() -> BatchCtx {
    if (uj == 0) {
      u = BatchCtx{};
      const int unit = gw + uk * tw;
      if (unit < total) {
        int lo = row_hint, hi = a.batch - 1;  // unit positions grow along the stream
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (s_prefix[mid] <= unit) lo = mid; else hi = mid - 1;
        }
        lo = uniform(lo);
        row_hint = lo;
        const int r = unit - uniform(s_prefix[lo]);
        const int span = HMAX ? r : (POW2 ? r >> a.hkv_log2 : r / a.Hkv);
        u.valid = 1;
        u.b = lo;
        u.t0 = span * a.U;
        u.len = uniform(s_len[lo]);
        u.g = HMAX ? 0 : r - span * a.Hkv;
        u.c0 = span * a.cpu;
        u.chunks_row = (u.len + a.chunk - 1) / a.chunk;
        u.qrow = uniform(s_qrow[lo]);
      }
      hj = 0;
      tj = 0;
    }
    BatchCtx c = u;
    if (HMAX) {  // one unit covers every KV head of its span, bph batches each
      c.g = hj;
      c.tg0 = tj * KB;
      if (++tj == bph) {
        tj = 0;
        ++hj;
      }
    } else {
      c.tg0 = uj * KB;
    }
    c.last = uj == bpu - 1;
    if (++uj == bpu) {
      uj = 0;
      ++uk;
    }
    return c;
  };

  // Every key load below is issued unconditionally, from wave-uniform bases
  // plus small per-lane offsets: lanes and batches with nothing to read use a
  // valid dummy address (row 0, or a clamped head / in-block row) and
  // compute() masks them.  Each batch therefore adds a fixed number of key
  // loads, and the wait for the batch being computed never drains the next
  // batch's keys.  q and the LSE are loaded only by a batch that starts a new
  // (row, KV head), before its keys (so a wait that covers them is one the
  // previous batch needed anyway); the other batches of the unit take them
  // from the batch computed just before (re-loading them every batch cost
  // about 5 us of a 57 us pass on 16 x 40k-token rows).
  //
  // pages_of() only issues the block-table loads (uniform: the group lies
  // inside one block); the page's address arithmetic waits for load(), one
  // computed batch later, so the scalar round trip overlaps that batch's
  // wait and maths.  Reading lanes past the row end stays inside the block.
  auto group_tok0 = [&](const BatchCtx& c, int i) { return c.t0 + (c.tg0 + i) * 16; };
  auto group_ok = [&](const BatchCtx& c, int i) {
    return c.valid && c.tg0 + i < a.ntu && group_tok0(c, i) < c.len;
  };
  auto pages_of = [&](const BatchCtx& c, int32_t (&kb)[KB]) {
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      kb[i] = 0;
      if (UNIFORM_PAGE) {
        const int tok0 = group_tok0(c, i);
        const int blk = POW2 ? tok0 >> a.bs_log2 : tok0 / a.block_size;
        kb[i] = scalar_load(a.bt + (group_ok(c, i) ? static_cast<int64_t>(c.b) * a.bt_stride + blk : 0));
      }
    }
  };
  auto page_base = [&](const BatchCtx& c, int i, int32_t page) -> int64_t {
    const int tok0 = group_tok0(c, i);
    const int in_block = POW2 ? tok0 & (a.block_size - 1) : tok0 % a.block_size;
    return group_ok(c, i) ? static_cast<int64_t>(page) * a.k_block_stride +
                                static_cast<int64_t>(in_block) * a.k_token_stride +
                                static_cast<int64_t>(c.g) * a.k_head_stride
                          : 0;
  };

  const int64_t lane_k = static_cast<int64_t>(col) * a.k_token_stride + kgrp * 8;
  const int q_head = min(col, a.G - 1);  // rows >= G read a real head; masked later

  int last_qrow = -1, last_g = -1;  // (query row, KV head) of the last loaded batch (wave-uniform)
  auto load = [&](const BatchCtx& c, const int32_t (&kb)[KB], Batch<KB, STEPS>& out) {
    out.c = c;
    out.fresh = c.qrow != last_qrow || c.g != last_g;
    last_qrow = c.qrow;
    last_g = c.g;
    if (out.fresh) {  // wave-uniform; issued before the keys
      const uint16_t* qh = a.q + static_cast<int64_t>(c.qrow) * a.q_stride + static_cast<int64_t>(c.g * a.G + q_head) * a.D +
                           kgrp * 8;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) out.q[s] = *reinterpret_cast<const Raw16*>(qh + 32 * s);
      if constexpr (!LSEFREE) {
        const float* lh = a.lse + static_cast<int64_t>(c.qrow) * a.lse_row_stride +
                          static_cast<int64_t>(c.g * a.G) * a.lse_head_stride;
#pragma unroll
        for (int i = 0; i < 4; ++i) out.lse[i] = lh[static_cast<int64_t>(min(4 * kgrp + i, a.G - 1)) * a.lse_head_stride];
      }
    }
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const uint16_t* krow;
      if (UNIFORM_PAGE) {
        krow = a.k + page_base(c, i, kb[i]) + lane_k;
      } else {
        const int tg = c.tg0 + i;
        const int tin = tg * 16 + col;
        const int tok = c.t0 + tin;
        const bool ok = c.valid && tg < a.ntu && tin < a.U && tok < c.len;
        const int64_t page = a.bt[ok ? static_cast<int64_t>(c.b) * a.bt_stride + tok / a.block_size : 0];
        const int64_t off = ok ? page * a.k_block_stride + static_cast<int64_t>(tok % a.block_size) * a.k_token_stride +
                                     static_cast<int64_t>(c.g) * a.k_head_stride
                               : 0;
        krow = a.k + off + kgrp * 8;
      }
#pragma unroll
      for (int s = 0; s < STEPS; ++s) out.k[i][s] = *reinterpret_cast<const Raw16*>(krow + 32 * s);
    }
  };
  // A batch of the same unit as the one just computed takes its q and LSE
  // from it (registers the computation has already waited for).
  auto inherit = [&](Batch<KB, STEPS>& next, const Batch<KB, STEPS>& done) {
    if (!next.fresh) {  // wave-uniform
#pragma unroll
      for (int s = 0; s < STEPS; ++s) next.q[s] = done.q[s];
#pragma unroll
      for (int i = 0; i < 4; ++i) next.lse[i] = done.lse[i];
    }
  };

  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // per chunk of the unit (head mean)
  float tmax[kMaxNtu];                  // per 16-token group (head max)
#pragma unroll
  for (int t = 0; t < kMaxNtu; ++t) tmax[t] = 0.f;
  // LSEFREE: the lane's running (max, sum) of query head 4 * kgrp + e over
  // its tokens of chunk `cur` of the unit, in log2 units.  A unit's token
  // groups run in order, so its chunks finish one after another: the pairs
  // are merged and stored when the chunk index moves on (registers only, no
  // per-chunk arrays).
  // One pair per token group slot of a batch keeps the slots' update chains
  // independent.
  float cm[KB][4], cz[KB][4];
#pragma unroll
  for (int i = 0; i < KB; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cm[i][e] = kNoMax;
      cz[i][e] = 0.f;
    }
  }
  int cur = 0;  // wave-uniform
  const float scale2 = a.scale * 1.44269504088896340736f;

  auto compute = [&](const Batch<KB, STEPS>& bt) {
    const BatchCtx& c = bt.c;
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const int tg = c.tg0 + i;
      if (tg >= a.ntu) continue;  // wave-uniform
      // Everything between the MFMA chain and the first read of its result
      // stays branch-free: the chunk index is one shift, computed up front.
      const int ci = (tg * 16) >> a.ci_shift;
      f32x4_t logit = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < STEPS; ++s) logit = mfma16x16x32<DT>(bt.q[s], bt.k[i][s], logit);
      const int tin = tg * 16 + col;
      const bool tok_ok = tin < a.U && c.t0 + tin < c.len;
      if (HMAX) {
        float m4 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (4 * kgrp + e < a.G && tok_ok) m4 = fmaxf(m4, __expf(logit[e] * a.scale - bt.lse[e]));
        }
        m4 = fmaxf(m4, __shfl_xor(m4, 16, 64));
        m4 = fmaxf(m4, __shfl_xor(m4, 32, 64));
#pragma unroll
        for (int t = 0; t < kMaxNtu; ++t) {
          tmax[t] = t == tg ? fmaxf(tmax[t], m4) : tmax[t];  // a select: tmax stays in registers
        }
      } else if constexpr (LSEFREE) {
        if (ci != cur) {  // wave-uniform
          flush_mass<KB, TAGGED>(a, c, cur, cm, cz, kgrp, col, tag);
          cur = ci;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          add_term(cm[i][e], cz[i][e], (4 * kgrp + e < a.G && tok_ok) ? logit[e] * scale2 : -INFINITY);
        }
      } else {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (4 * kgrp + e < a.G && tok_ok) s += __expf(logit[e] * a.scale - bt.lse[e]);
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) acc[cc] += cc == ci ? s : 0.f;
      }
    }
    if (!c.last) return;
    const int chunks_row = c.chunks_row;
    if (HMAX) {
      for (int cc = 0; cc < a.cpu; ++cc) {
        float s = 0.f;
#pragma unroll
        for (int t = 0; t < kMaxNtu; ++t) {
          if (kgrp == 0 && t < a.ntu && (t * 16) / a.chunk == cc && t * 16 + col < a.U &&
              c.t0 + t * 16 + col < c.len) {
            s += tmax[t];
          }
        }
        s = wave_sum(s);
        const int ch = c.c0 + cc;
        if (lane == 0 && ch < chunks_row) {
          const int n_valid = min(a.chunk, c.len - ch * a.chunk);
          a.out[static_cast<int64_t>(c.b) * a.out_stride + ch] = s / static_cast<float>(n_valid);
        }
      }
#pragma unroll
      for (int t = 0; t < kMaxNtu; ++t) tmax[t] = 0.f;
    } else if constexpr (LSEFREE) {
      flush_mass<KB, TAGGED>(a, c, cur, cm, cz, kgrp, col, tag);
      cur = 0;
    } else {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        if (cc < a.cpu) {
          const float s = wave_sum_to_lane63(acc[cc]);
          const int ch = c.c0 + cc;
          if (lane == 63 && ch < chunks_row) {
            const int64_t at = (static_cast<int64_t>(c.b) * a.max_chunks + ch) * a.Hkv + c.g;
            if constexpr (TAGGED) {
              // A coherent store that needs no wait: the value carries the
              // launch's tag, so a reader polling it needs no other signal.
              const uint64_t v = (static_cast<uint64_t>(tag) << 32) | __float_as_uint(s);
              __hip_atomic_store(a.tagged + at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
              a.partial[at] = s;
            }
          }
        }
        acc[cc] = 0.f;
      }
    }
  };

  // Three-stage pipeline, unrolled by two so every buffer index is static.
  // Per half: vector loads for batch n+1 (their block-table entries arrived
  // a half earlier), then the block-table lookups for n+2, then the maths of
  // batch n.  Scalar loads complete out of order, so the lookups are issued
  // after the loads that consume the previous ones.
  BatchCtx cx0 = next_ctx();
  BatchCtx cx1 = next_ctx();
  int32_t pg0[KB], pg1[KB];
  pages_of(cx0, pg0);
  pages_of(cx1, pg1);
  Batch<KB, STEPS> d0, d1;
  load(cx0, pg0, d0);
  for (;;) {
    if (!d0.c.valid) break;
    load(cx1, pg1, d1);
    cx0 = next_ctx();
    pages_of(cx0, pg0);
    compute(d0);
    inherit(d1, d0);
    if (!d1.c.valid) break;
    load(cx0, pg0, d0);
    cx1 = next_ctx();
    pages_of(cx1, pg1);
    compute(d1);
    inherit(d0, d1);
  }
}

// ---- Each query head's LSE from a row's mass words ------------------------
// Both the kernel chain (lse_finalize_kernel) and the single launch's
// selectors merge a row's mass words with this thread layout and these merge
// steps, so both give the same bits.
//
// One KV group's G heads over the row's chunks, kThreads threads.  hp heads
// per thread: 2 (`wide`, G even: one 16-byte read covers both) or 1.
// P = G / hp phases, tpp threads per phase (a power of two, tpp * P <=
// kThreads).  Thread (ph, j) adds the masses of chunks j, j + tpp, j + 2 tpp,
// ... in that order (add_term); the lanes of one phase then merge by xor
// shuffles (lane distances lstep .. lstep * lanes / 2), and the waves'
// results are merged in LDS in wave order.  How the loads are batched does
// not change any of these sums.  With P a power of two consecutive lanes
// take consecutive phases, so a wave reads whole runs of a chunk's words;
// otherwise each phase takes tpp adjacent lanes.
constexpr int kLseLoads = 16;
// The merge takes two heads per thread when the words are 16-byte aligned.
inline int lse_words_wide(const void* mw) { return (reinterpret_cast<uintptr_t>(mw) & 15u) == 0 ? 1 : 0; }
struct LseLayout {
  int hp, P, tpp, ph, j, lstep, lanes;
  bool inter;
};
__device__ __forceinline__ LseLayout lse_layout(int G, int wide, int t) {
  LseLayout l;
  l.hp = wide && G % 2 == 0 ? 2 : 1;
  l.P = G / l.hp;
  l.inter = (l.P & (l.P - 1)) == 0;
  l.tpp = 1;
  while (l.tpp * 2 * l.P <= kThreads) l.tpp *= 2;
  l.ph = l.inter ? (t & (l.P - 1)) : t / l.tpp;
  l.j = l.inter ? t / l.P : t % l.tpp;
  l.lstep = l.inter ? l.P : 1;
  l.lanes = l.inter ? 64 / l.P : (l.tpp < 64 ? l.tpp : 64);
  return l;
}

// A thread's running sums of its hp heads, in log2 units.
struct LseAcc {
  float m0 = kNoMax, z0 = 0.f, m1 = kNoMax, z1 = 0.f;
  __device__ __forceinline__ void add(uint64_t w0, uint64_t w1, int hp) {
    add_term(m0, z0, mass_of(w0));
    if (hp == 2) add_term(m1, z1, mass_of(w1));
  }
};

// Ends one group's merge: the lane shuffles, then the waves' results through
// s_m / s_z ([2][kThreads] floats of LDS the caller lends; a barrier on each
// side).  Returns head t's natural-log LSE for t < G (-inf for a head with no
// chunk).
__device__ __forceinline__ float lse_finish(const LseLayout& l, LseAcc acc, int G, float (*s_m)[kThreads],
                                            float (*s_z)[kThreads]) {
  const int t = threadIdx.x;
  for (int off = l.lstep; off < l.lstep * l.lanes; off <<= 1) {
    merge_mz(acc.m0, acc.z0, __shfl_xor(acc.m0, off, 64), __shfl_xor(acc.z0, off, 64));
    if (l.hp == 2) merge_mz(acc.m1, acc.z1, __shfl_xor(acc.m1, off, 64), __shfl_xor(acc.z1, off, 64));
  }
  s_m[0][t] = acc.m0;
  s_z[0][t] = acc.z0;
  s_m[1][t] = acc.m1;
  s_z[1][t] = acc.z1;
  __syncthreads();
  float lse = -INFINITY;
  if (t < G) {
    // Head t is half t % hp of phase t / hp; one merged pair per wave of the
    // phase: lane (phase) of every wave, or the first lane of each 64-lane
    // block of the phase's tpp lanes.
    const int q = t / l.hp, half = t % l.hp;
    float mh = -INFINITY, zh = 0.f;
    for (int k = 0; k < l.tpp; k += l.lanes) {
      const int at = l.inter ? (k / l.lanes) * 64 + q : q * l.tpp + k;
      merge_mz(mh, zh, s_m[half][at], s_z[half][at]);
    }
    const float lse2 = zh > 0.f ? mh + __log2f(zh) : -INFINITY;
    lse = lse2 * 0.69314718055994530942f;
  }
  __syncthreads();
  return lse;
}

// The exponent base of a head's chunk shares: its LSE as written (natural
// log, fp32), in log2 units.
__device__ __forceinline__ float lse_base2(float lse) { return lse * 1.44269504088896340736f; }

// One head's share of a chunk's score, 2^(M - lse2), added to a KV group's
// running sum (heads in order, from 0): nothing for a chunk or head without
// mass.
__device__ __forceinline__ float add_share(float sum, float mass, float lse2) {
  return mass != -INFINITY && lse2 != -INFINITY ? sum + __builtin_amdgcn_exp2f(mass - lse2) : sum;
}

}  // namespace score
}  // namespace ds355
