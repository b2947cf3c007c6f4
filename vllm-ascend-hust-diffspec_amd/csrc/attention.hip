// Draft decode attention over the working cache's capacity view.
//
// Counterpart of DiffSpecDraftCache.forward_attention's linear path:
// diffspec/runtime.py:2024-2077 (CPU loop) and :2079-2134 (one batched NPU
// fused-attention call over the [slot, head, token_budget, head_dim] view with
// per-row valid lengths).  For each row r with slot s and local position p:
//   working_key[s, :, p] = key[r], working_value[s, :, p] = value[r],
//   working_lens[s] = p + 1,
//   out[r, h] = softmax(scale * q[r, h] . K[s, h / G, 0..p]) V[s, h / G, 0..p]
// in fp32, and out rows past the batch are zero.
//
// Work split: one workgroup per (row, KV head, block of up to 16 query heads
// of that KV head's group, span of tokens).  Each of its 4 waves walks
// 16-token tiles of its quarter of the span:
//   scores  S[t][g] = K[t] . Q[g]     one 16x16x32 bf16/fp16 MFMA per 32 of
//                                     head_dim, K as the A operand (lane owns
//                                     token t = lane % 16), Q as B (lane owns
//                                     query g = lane % 16);
//   softmax online per query g (lane column), rows of the S tile are tokens
//                                     4 * (lane / 16) + i;
//   output  O^T[d][g] += V^T[d][t] P^T[t][g]   16x16x4 fp32 MFMAs: for the
//                                     i-th row of every lane's S tile the k
//                                     index lane / 16 is token 4 * (lane / 16)
//                                     + i, so the B operand is the lane's own
//                                     probability; head_dim column m of block
//                                     j is d = J * m + j (J = D / 16), so the
//                                     A operand is one contiguous J-element
//                                     vector of V's row, and each lane ends
//                                     with the D / 4 contiguous outputs
//                                     [4J * (lane / 16), 4J * (lane / 16 + 1))
//                                     of query g.
// Probabilities stay fp32 (the reference's softmax is fp32 and multiplies
// fp32 V).  The four waves merge in LDS.  A row that fits one span writes its
// output directly; longer rows write per-span partials (running max, sum and
// unnormalised output), and the last span workgroup to finish merges them.
//
// Hand-over between workgroups needs no waiting on other workgroups' progress
// and no cache flushes: partial values are stored as 64-bit words
// (tag << 32 | fp32 bits) with device-scope stores, tag = launch epoch + 1;
// the merging workgroup reads them with device-scope loads and re-reads any
// word whose tag is not yet the launch's (its writer has already counted
// itself, so the store is in flight).  The last merging workgroup advances the
// epoch, which keeps graph replays and workspace reuse safe.  The new token's
// K/V is read from the input rows (its working-cache slot is written by the
// same launch), and working_lens[slot] is written by the last workgroup of
// the row to read it, so positions may come from working_lens itself.
#include "ds355_common.h"

namespace ds355 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreadsA = 256;
constexpr int kWavesA = kThreadsA / 64;
constexpr int kTileT = 16;        // tokens per MFMA tile
constexpr int kGroupQ = 16;       // query heads per workgroup (MFMA N)
constexpr int kMaxUnitsPerRow = 128;  // KV heads x query blocks
constexpr uint32_t kSpinA = 1u << 20;
constexpr float kLog2e = 1.44269504088896340736f;

// Workspace layout (bytes): header, row counters, unit counters, partials.
enum { kHdrEpoch = 0, kHdrCombined = 1, kHdrStatus = 2 };
constexpr size_t kHeaderBytes = 256;
constexpr size_t kRowCountOffset = kHeaderBytes;
constexpr size_t kUnitCountOffset = kRowCountOffset + sizeof(uint32_t) * kMaxRows;
constexpr size_t kPartialOffset = kUnitCountOffset + sizeof(uint32_t) * kMaxRows * kMaxUnitsPerRow;
constexpr uint32_t kStatusPosition = 1;  // a row's slot or position was out of range
constexpr uint32_t kStatusPartials = 2;  // a merge stopped waiting for a partial

template <int D>
struct AttnShape {
  static constexpr int kTiles = D <= 128 ? 4 : 2;          // tiles per wave
  static constexpr int kSpan = kWavesA * kTiles * kTileT;  // tokens per workgroup
  static constexpr int kSteps = D / 32;                    // score MFMAs per tile
  static constexpr int kJ = D / 16;                        // output column blocks
  static constexpr int kRow = D + 2;                       // partial words per query
};

struct AttnArgs {
  const void* q;
  int64_t q_row, q_head;
  const void* k_in;
  int64_t k_row, k_head;
  const void* v_in;
  int64_t v_row, v_head;
  void* out;
  int64_t o_row, o_head;
  void* work_k;
  void* work_v;
  int32_t* working_lens;
  const int32_t* slots;
  const int32_t* positions;
  int rows, out_rows, num_slots, hq, hkv, group, qblocks, budget, splits;
  float scale;
  uint32_t* header;
  uint32_t* row_count;
  uint32_t* unit_count;
  uint64_t* partials;
};

template <int DT>
__device__ __forceinline__ f32x4 mfma_scores(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_scores<DS_BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_scores<DS_FP16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// Element e of a packed pair word to fp32.
template <int DT>
__device__ __forceinline__ float unpack(uint32_t w, int half) {
  if (DT == DS_BF16) return __uint_as_float(half ? (w & 0xffff0000u) : (w << 16));
  return f16_to_f32(static_cast<uint16_t>(half ? (w >> 16) : (w & 0xffffu)));
}

__device__ __forceinline__ u32x4 load16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// J consecutive 16-bit elements (J = 4, 8 or 16) as J / 2 words.
template <int J>
__device__ __forceinline__ void load_words(const uint16_t* p, uint32_t (&w)[J / 2]) {
  if constexpr (J == 4) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int h = 0; h < J / 8; ++h) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + 8 * h);
      w[4 * h] = v.x; w[4 * h + 1] = v.y; w[4 * h + 2] = v.z; w[4 * h + 3] = v.w;
    }
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint64_t tagged(uint32_t tag, float v) {
  return (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
}

__device__ __forceinline__ void raise_status(const AttnArgs& a, uint32_t bit) {
  __hip_atomic_fetch_or(a.header + kHdrStatus, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Value of a tagged partial word once its tag is this launch's.  The writer
// counted itself after issuing the store, so the wait is for a store in
// flight; it is bounded all the same, and after one expiry the thread stops
// waiting (NaN results, status bit set).
__device__ __forceinline__ float settle(const AttnArgs& a, const uint64_t* p, uint64_t v, uint32_t tag,
                                        bool& expired) {
  uint32_t spins = 0;
  while (static_cast<uint32_t>(v >> 32) != tag) {
    if (expired || ++spins > kSpinA) {
      if (!expired) raise_status(a, kStatusPartials);
      expired = true;
      return __uint_as_float(0x7fc00000u);
    }
    __builtin_amdgcn_s_sleep(2);
    v = coherent_load(p);
  }
  return __uint_as_float(static_cast<uint32_t>(v));
}

// Zero out[row, head0 .. head0 + count) (padding rows and rows with a bad position).
template <int D>
__device__ __forceinline__ void zero_heads(const AttnArgs& a, int row, int head0, int count) {
  uint16_t* o = static_cast<uint16_t*>(a.out) + static_cast<int64_t>(row) * a.o_row;
  const int chunks = count * (D / 8);
  for (int c = threadIdx.x; c < chunks; c += kThreadsA) {
    const int g = c / (D / 8), e = c % (D / 8);
    *reinterpret_cast<u32x4*>(o + static_cast<int64_t>(head0 + g) * a.o_head + 8 * e) = u32x4{0, 0, 0, 0};
  }
}

template <int DT, int D>
__global__ __launch_bounds__(kThreadsA, 2) void draft_attention_kernel(AttnArgs a) {
  using S = AttnShape<D>;
  constexpr int J = S::kJ;
  __shared__ float s_m[kWavesA][kGroupQ];
  __shared__ float s_l[kWavesA][kGroupQ];
  __shared__ float s_acc[kWavesA - 1][kGroupQ][D + 4];
  __shared__ int s_pos;
  __shared__ uint32_t s_tag;
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int quad = lane >> 4;
  int b = blockIdx.x;
  const int split = b % a.splits;
  b /= a.splits;
  const int qb = b % a.qblocks;
  b /= a.qblocks;
  const int kvh = b % a.hkv;
  const int row = b / a.hkv;
  const int g0 = qb * kGroupQ;
  const int gcount = min(kGroupQ, a.group - g0);
  const int head0 = kvh * a.group + g0;

  if (row >= a.rows) {  // padding row: zero once
    if (split == 0) zero_heads<D>(a, row, head0, gcount);
    return;
  }

  // Thread 0 reads the row's position, then counts this workgroup as one of
  // the row's readers; the waitcnt makes the read complete before the count,
  // so the last reader may overwrite working_lens[slot].
  const int slot = scalar_load(a.slots + row);
  uint32_t row_old = 0;
  if (threadIdx.x == 0) {
    int pos = -1;
    if (slot >= 0 && slot < a.num_slots) pos = a.positions ? a.positions[row] : a.working_lens[slot];
    const uint32_t epoch = coherent_load(a.header + kHdrEpoch);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    s_pos = (pos >= 0 && pos < a.budget) ? pos : -1;
    s_tag = epoch + 1;
    row_old = __hip_atomic_fetch_add(a.row_count + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const int pos = s_pos;
  const uint32_t tag = s_tag;
  const bool valid = pos >= 0;
  const int n = valid ? pos + 1 : 0;
  const int active = valid ? (n + S::kSpan - 1) / S::kSpan : 1;

  // The last of the row's workgroups to read the position publishes p + 1.
  auto finish_row = [&]() {
    if (threadIdx.x == 0 && row_old == static_cast<uint32_t>(a.hkv * a.qblocks * a.splits - 1)) {
      coherent_store(a.row_count + row, 0u);
      if (valid) a.working_lens[slot] = pos + 1;
      else raise_status(a, kStatusPosition);
    }
  };
  // Every (row, KV head, query block) has one merging workgroup; the last of
  // them advances the epoch.
  auto finish_unit = [&]() {
    if (threadIdx.x == 0) {
      const uint32_t total = static_cast<uint32_t>(a.rows * a.hkv * a.qblocks);
      const uint32_t old = __hip_atomic_fetch_add(a.header + kHdrCombined, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if (old == total - 1) {
        coherent_store(a.header + kHdrCombined, 0u);
        coherent_store(a.header + kHdrEpoch, tag);
      }
    }
  };

  if (split >= active) {
    finish_row();
    return;
  }
  if (!valid) {  // bad slot or position: zero output, touch nothing else
    zero_heads<D>(a, row, head0, gcount);
    finish_unit();
    finish_row();
    return;
  }

  const int64_t work_base = (static_cast<int64_t>(slot) * a.hkv + kvh) * a.budget * D;
  const uint16_t* kw = static_cast<const uint16_t*>(a.work_k) + work_base;
  const uint16_t* vw = static_cast<const uint16_t*>(a.work_v) + work_base;
  const uint16_t* kin = static_cast<const uint16_t*>(a.k_in) + row * a.k_row + kvh * a.k_head;
  const uint16_t* vin = static_cast<const uint16_t*>(a.v_in) + row * a.v_row + kvh * a.v_head;

  // The new token goes into the working cache (nobody reads that slot here).
  if (qb == 0 && split == pos / S::kSpan && threadIdx.x < D / 4) {
    const int e = threadIdx.x % (D / 8);
    const bool is_v = threadIdx.x >= D / 8;
    uint16_t* dst = static_cast<uint16_t*>(is_v ? a.work_v : a.work_k) + work_base + static_cast<int64_t>(pos) * D;
    *reinterpret_cast<u32x4*>(dst + 8 * e) = load16((is_v ? vin : kin) + 8 * e);
  }

  // Query block as the B operand of the score MFMAs: lane (quad, col) holds
  // q[head0 + col][32 i + 8 quad .. + 8].
  u32x4 qv[S::kSteps];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + row * a.q_row + (head0 + col) * a.q_head + 8 * quad;
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) qv[i] = col < gcount ? load16(qp + 32 * i) : u32x4{0, 0, 0, 0};
  }

  f32x4 acc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;
  const float c = a.scale * kLog2e;
  const int t0 = split * S::kSpan + wave * S::kTiles * kTileT;

  // One tile's operands: K rows for the score MFMAs, V rows for the output.
  struct Tile {
    u32x4 k[S::kSteps];
    uint32_t v[4][J / 2];
  };
  auto load_tile = [&](Tile& T, int tb) {
    const int tk = tb + col;
    const uint16_t* p = (tk == pos ? kin : kw + static_cast<int64_t>(tk) * D) + 8 * quad;
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) T.k[i] = tk < n ? load16(p + 32 * i) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tb + 4 * quad + r;
      if (t < n) {
        load_words<J>((t == pos ? vin : vw + static_cast<int64_t>(t) * D) + J * col, T.v[r]);
      } else {
#pragma unroll
        for (int w = 0; w < J / 2; ++w) T.v[r][w] = 0;
      }
    }
  };
  auto compute_tile = [&](const Tile& T, int tb) {
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) s = mfma_scores<DT>(T.k[i], qv[i], s);
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (tb + 4 * quad + i < n) ? s[i] * c : -INFINITY;
    float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mn = fmaxf(m, tmax);
    const float alpha = fast_exp2(m - mn);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(x[i] - mn);
    lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m = mn;
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] *= alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int j = 0; j < J; ++j) {
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(unpack<DT>(T.v[r][j >> 1], j & 1), p[r], acc[j], 0, 0, 0);
      }
    }
  };

  // Two tiles in flight: the next tile's loads are issued before the current
  // tile is computed.
  if (t0 < n) {
    Tile cur, nxt;
    load_tile(cur, t0);
#pragma unroll 1
    for (int k = 0; k < S::kTiles; k += 2) {
      const int tb = t0 + k * kTileT;
      const bool more = k + 1 < S::kTiles && tb + kTileT < n;
      if (more) load_tile(nxt, tb + kTileT);
      compute_tile(cur, tb);
      if (!more) break;
      const bool more2 = k + 2 < S::kTiles && tb + 2 * kTileT < n;
      if (more2) load_tile(cur, tb + 2 * kTileT);
      compute_tile(nxt, tb + kTileT);
      if (!more2) break;
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // Merge the four waves: common max, rescale, sum in wave order.
  if (quad == 0) {
    s_m[wave][col] = m;
    s_l[wave][col] = lsum;
  }
  __syncthreads();
  float mx = s_m[0][col];
#pragma unroll
  for (int w = 1; w < kWavesA; ++w) mx = fmaxf(mx, s_m[w][col]);
  float total_l = 0.f;
#pragma unroll
  for (int w = 0; w < kWavesA; ++w) total_l += s_l[w][col] * fast_exp2(s_m[w][col] - mx);
  const float f = fast_exp2(m - mx);
  const int d0 = 4 * J * quad;  // lane's outputs: d = d0 + J * i + j
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < J; ++j) s_acc[wave - 1][col][d0 + J * i + j] = acc[j][i] * f;
    }
  }
  __syncthreads();

  if (active == 1) {
    if (wave == 0 && col < gcount) {
      const float inv = 1.f / total_l;
      uint16_t* o = static_cast<uint16_t*>(a.out) + row * a.o_row + (head0 + col) * a.o_head + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t w[J / 2];
#pragma unroll
        for (int j = 0; j < J; j += 2) {
          float v0 = acc[j][i] * f, v1 = acc[j + 1][i] * f;
#pragma unroll
          for (int ww = 0; ww < kWavesA - 1; ++ww) {
            v0 += s_acc[ww][col][d0 + J * i + j];
            v1 += s_acc[ww][col][d0 + J * i + j + 1];
          }
          w[j / 2] = static_cast<uint32_t>(Elem<DT>::store(v0 * inv)) |
                     (static_cast<uint32_t>(Elem<DT>::store(v1 * inv)) << 16);
        }
        if constexpr (J == 4) {
          *reinterpret_cast<u32x2*>(o + J * i) = u32x2{w[0], w[1]};
        } else {
#pragma unroll
          for (int h = 0; h < J / 8; ++h) {
            *reinterpret_cast<u32x4*>(o + J * i + 8 * h) = u32x4{w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]};
          }
        }
      }
    }
    finish_unit();
    finish_row();
    return;
  }

  // Several spans: publish this span's partial, the last one merges.
  const int unit = (row * a.hkv + kvh) * a.qblocks + qb;
  uint64_t* part_base = a.partials + static_cast<int64_t>(unit) * a.splits * kGroupQ * S::kRow;
  if (wave == 0) {
    if (col < gcount) {
      uint64_t* pr = part_base + (static_cast<int64_t>(split) * kGroupQ + col) * S::kRow;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
          float v = acc[j][i] * f;
#pragma unroll
          for (int ww = 0; ww < kWavesA - 1; ++ww) v += s_acc[ww][col][d0 + J * i + j];
          coherent_store(pr + d0 + J * i + j, tagged(tag, v));
        }
      }
      if (quad == 0) {
        coherent_store(pr + D, tagged(tag, mx));
        coherent_store(pr + D + 1, tagged(tag, total_l));
      }
    }
    if (lane == 0) {
      const uint32_t old = __hip_atomic_fetch_add(a.unit_count + static_cast<int64_t>(row) * kMaxUnitsPerRow +
                                                      kvh * a.qblocks + qb,
                                                  1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = old == static_cast<uint32_t>(active - 1);
    }
  }
  __syncthreads();
  if (!s_last) {
    finish_row();
    return;
  }

  // Merge: thread -> (query g, 4 consecutive outputs), spans in order, in
  // groups of kGroupS spans whose words are all requested before any is used.
  constexpr int kChunks = D / 4;
  constexpr int kGroupS = 4;
  bool expired = false;
  for (int item = threadIdx.x; item < gcount * kChunks; item += kThreadsA) {
    const int g = item / kChunks;
    const int e = 4 * (item % kChunks);
    float run_m = -INFINITY, run_l = 0.f;
    float run[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < active; s0 += kGroupS) {
      const int cnt = min(kGroupS, active - s0);
      uint64_t wm[kGroupS], wl[kGroupS], wv[kGroupS][4];
#pragma unroll
      for (int u = 0; u < kGroupS; ++u) {
        if (u < cnt) {
          const uint64_t* pr = part_base + (static_cast<int64_t>(s0 + u) * kGroupQ + g) * S::kRow;
          wm[u] = coherent_load(pr + D);
          wl[u] = coherent_load(pr + D + 1);
#pragma unroll
          for (int v = 0; v < 4; ++v) wv[u][v] = coherent_load(pr + e + v);
        }
      }
      float gm = run_m;
      float vm[kGroupS];
#pragma unroll
      for (int u = 0; u < kGroupS; ++u) {
        if (u < cnt) {
          const uint64_t* pr = part_base + (static_cast<int64_t>(s0 + u) * kGroupQ + g) * S::kRow;
          vm[u] = settle(a, pr + D, wm[u], tag, expired);
          gm = fmaxf(gm, vm[u]);
        }
      }
      const float rescale = fast_exp2(run_m - gm);
      run_l *= rescale;
#pragma unroll
      for (int v = 0; v < 4; ++v) run[v] *= rescale;
#pragma unroll
      for (int u = 0; u < kGroupS; ++u) {
        if (u < cnt) {
          const uint64_t* pr = part_base + (static_cast<int64_t>(s0 + u) * kGroupQ + g) * S::kRow;
          const float w = fast_exp2(vm[u] - gm);
          run_l += settle(a, pr + D + 1, wl[u], tag, expired) * w;
#pragma unroll
          for (int v = 0; v < 4; ++v) run[v] += settle(a, pr + e + v, wv[u][v], tag, expired) * w;
        }
      }
      run_m = gm;
    }
    const float inv = 1.f / run_l;
    uint16_t* o = static_cast<uint16_t*>(a.out) + row * a.o_row + (head0 + g) * a.o_head + e;
    const uint32_t w0 = static_cast<uint32_t>(Elem<DT>::store(run[0] * inv)) |
                        (static_cast<uint32_t>(Elem<DT>::store(run[1] * inv)) << 16);
    const uint32_t w1 = static_cast<uint32_t>(Elem<DT>::store(run[2] * inv)) |
                        (static_cast<uint32_t>(Elem<DT>::store(run[3] * inv)) << 16);
    *reinterpret_cast<u32x2*>(o) = u32x2{w0, w1};
  }
  if (threadIdx.x == 0) {
    coherent_store(a.unit_count + static_cast<int64_t>(row) * kMaxUnitsPerRow + kvh * a.qblocks + qb, 0u);
  }
  finish_unit();
  finish_row();
}

template <int DT, int D>
int launch_attention(hipStream_t stream, const AttnArgs& a) {
  const int64_t grid = static_cast<int64_t>(a.out_rows) * a.hkv * a.qblocks * a.splits;
  draft_attention_kernel<DT, D><<<static_cast<unsigned>(grid), kThreadsA, 0, stream>>>(a);
  return check_launch("ds_draft_attention");
}

int span_for(int head_dim) { return head_dim <= 128 ? kWavesA * 4 * kTileT : kWavesA * 2 * kTileT; }

size_t attention_workspace_bytes(int rows, int num_q_heads, int num_kv_heads, int head_dim, int token_budget) {
  if (rows <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || token_budget <= 0) return 0;
  if (num_q_heads % num_kv_heads) return 0;
  const int group = num_q_heads / num_kv_heads;
  const int qblocks = (group + kGroupQ - 1) / kGroupQ;
  const int splits = (token_budget + span_for(head_dim) - 1) / span_for(head_dim);
  const size_t partial = static_cast<size_t>(rows) * num_kv_heads * qblocks * splits * kGroupQ * (head_dim + 2) *
                         sizeof(uint64_t);
  return kPartialOffset + partial;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int draft_attention_impl(hipStream_t stream, int dtype, const void* query, int64_t q_row, int64_t q_head,
                         const void* key, int64_t k_row, int64_t k_head, const void* value, int64_t v_row,
                         int64_t v_head, void* out, int64_t o_row, int64_t o_head, void* working_key,
                         void* working_value, int32_t* working_lens, const int32_t* slots,
                         const int32_t* positions, int rows, int out_rows, int num_slots, int num_q_heads,
                         int num_kv_heads, int head_dim, int token_budget, float scale, void* workspace,
                         size_t workspace_bytes) {
  DS_REQUIRE(rows >= 0 && out_rows >= rows, "output rows must cover the pending rows");
  DS_REQUIRE(num_slots > 0 && token_budget > 0 && head_dim > 0, "working cache shape must be positive");
  DS_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
             "query heads must be a positive multiple of KV heads");
  DS_REQUIRE(rows <= num_slots, "more pending rows than working-cache slots");
  DS_SUPPORTED(dtype == DS_BF16 || dtype == DS_FP16, "draft attention runs on BF16 or FP16 tensors");
  DS_SUPPORTED(head_dim == 64 || head_dim == 128 || head_dim == 256, "draft attention head_dim must be 64, 128 or 256");
  DS_SUPPORTED(out_rows <= kMaxRows, "at most %d output rows per launch (got %d)", kMaxRows, out_rows);
  const int group = num_q_heads / num_kv_heads;
  const int qblocks = (group + kGroupQ - 1) / kGroupQ;
  DS_SUPPORTED(num_kv_heads * qblocks <= kMaxUnitsPerRow, "too many KV heads x query blocks (%d > %d)",
               num_kv_heads * qblocks, kMaxUnitsPerRow);
  if (out_rows == 0) return clear_error();
  DS_REQUIRE(query && out && (rows == 0 || (key && value && working_key && working_value && working_lens && slots)),
             "null tensor pointer");
  DS_REQUIRE(workspace, "draft attention needs a workspace");
  const size_t need = attention_workspace_bytes(rows > 0 ? rows : 1, num_q_heads, num_kv_heads, head_dim,
                                                token_budget);
  DS_REQUIRE(workspace_bytes >= need, "attention workspace too small: %zu bytes, need %zu", workspace_bytes, need);
  DS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "workspace must be 256-byte aligned");
  // 16-byte vector accesses: every row and head start must be 16-byte aligned.
  DS_REQUIRE(aligned16(query) && aligned16(out) && q_row % 8 == 0 && q_head % 8 == 0 && o_row % 8 == 0 &&
                 o_head % 8 == 0,
             "query and output rows and heads must start on 16-byte boundaries");
  DS_REQUIRE(rows == 0 || (aligned16(key) && aligned16(value) && aligned16(working_key) &&
                           aligned16(working_value) && k_row % 8 == 0 && k_head % 8 == 0 && v_row % 8 == 0 &&
                           v_head % 8 == 0),
             "key, value and working caches must start rows and heads on 16-byte boundaries");

  AttnArgs a{};
  a.q = query; a.q_row = q_row; a.q_head = q_head;
  a.k_in = key; a.k_row = k_row; a.k_head = k_head;
  a.v_in = value; a.v_row = v_row; a.v_head = v_head;
  a.out = out; a.o_row = o_row; a.o_head = o_head;
  a.work_k = working_key; a.work_v = working_value;
  a.working_lens = working_lens; a.slots = slots; a.positions = positions;
  a.rows = rows; a.out_rows = out_rows; a.num_slots = num_slots;
  a.hq = num_q_heads; a.hkv = num_kv_heads; a.group = group; a.qblocks = qblocks;
  a.budget = token_budget;
  a.splits = (token_budget + span_for(head_dim) - 1) / span_for(head_dim);
  a.scale = scale;
  char* ws = static_cast<char*>(workspace);
  a.header = reinterpret_cast<uint32_t*>(ws);
  a.row_count = reinterpret_cast<uint32_t*>(ws + kRowCountOffset);
  a.unit_count = reinterpret_cast<uint32_t*>(ws + kUnitCountOffset);
  a.partials = reinterpret_cast<uint64_t*>(ws + kPartialOffset);

#define DS_ATTN_CASE(DTV, DV) \
  if (dtype == DTV && head_dim == DV) return launch_attention<DTV, DV>(stream, a);
  DS_ATTN_CASE(DS_BF16, 64) DS_ATTN_CASE(DS_BF16, 128) DS_ATTN_CASE(DS_BF16, 256)
  DS_ATTN_CASE(DS_FP16, 64) DS_ATTN_CASE(DS_FP16, 128) DS_ATTN_CASE(DS_FP16, 256)
#undef DS_ATTN_CASE
  return set_error(DS_ERR_UNSUPPORTED, "unsupported draft attention shape");
}

}  // namespace
}  // namespace ds355

extern "C" size_t ds_draft_attention_workspace_bytes(int batch_rows, int num_q_heads, int num_kv_heads,
                                                     int head_dim, int token_budget) {
  return ds355::attention_workspace_bytes(batch_rows, num_q_heads, num_kv_heads, head_dim, token_budget);
}

extern "C" int ds_draft_attention(ds_stream_t stream, int dtype, const void* query, int64_t q_row_stride,
                                  int64_t q_head_stride, const void* key, int64_t k_row_stride,
                                  int64_t k_head_stride, const void* value, int64_t v_row_stride,
                                  int64_t v_head_stride, void* out, int64_t o_row_stride, int64_t o_head_stride,
                                  void* working_key, void* working_value, int32_t* working_lens,
                                  const int32_t* slots, const int32_t* positions, int rows, int out_rows,
                                  int num_slots, int num_q_heads, int num_kv_heads, int head_dim, int token_budget,
                                  float scale, void* workspace, size_t workspace_bytes) {
  return ds355::draft_attention_impl(reinterpret_cast<hipStream_t>(stream), dtype, query, q_row_stride,
                                     q_head_stride, key, k_row_stride, k_head_stride, value, v_row_stride,
                                     v_head_stride, out, o_row_stride, o_head_stride, working_key, working_value,
                                     working_lens, slots, positions, rows, out_rows, num_slots, num_q_heads,
                                     num_kv_heads, head_dim, token_budget, scale, workspace, workspace_bytes);
}
