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
// output directly; in a longer row every span but the last writes its
// partial (running max, sum and unnormalised output) and exits, and the last
// span's workgroup merges them with its own.
//
// Hand-over between workgroups needs no cache flushes and no counting:
// partial values are stored as 64-bit words (tag << 32 | fp32 bits) with
// device-scope stores, tag = launch epoch + 1, and the merging workgroup
// re-reads (device-scope loads) any word whose tag is not yet the launch's.
// It only waits for workgroups of lower index (the row's earlier spans),
// which are dispatched before it, so the wait ends whether or not the grid is
// resident at once; it is bounded all the same.  The last merging workgroup
// advances the epoch, which keeps graph replays and workspace reuse safe.
// The new token's K/V is read from the input rows (its working-cache slot is
// written by the same launch), and working_lens[slot] is written by the last
// workgroup of the row to read it, so positions may come from working_lens
// itself.  Waits in this kernel are LDS-only barriers and the merge's tag
// checks: the row count and the epoch load stay in flight behind the loads.
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
constexpr int kGroupS = 8;      // other spans merged per round trip
constexpr uint32_t kSpinA = 1u << 20;
constexpr float kLog2e = 1.44269504088896340736f;

// Workspace layout (bytes): a 256-byte header (epoch, status); a fixed
// region of kMaxUnits 32-bit span counters, one per (row, KV head, query
// block), 0 between launches (a shape-independent place, so a launch of
// another shape never reads other words as counters); one tagged "seen"
// word per workgroup of the pending rows (64-bit, tag << 32 | value, so a
// launch of another shape finds only older tags); then the fp32 partial
// results of every span.
constexpr int kMaxUnits = 65536;
constexpr size_t kCounterBytes = kMaxUnits * sizeof(uint32_t);
enum { kHdrEpoch = 0, kHdrStatus = 2 };
constexpr size_t kHeaderBytes = 256;
constexpr uint32_t kStatusPosition = 1;  // a row's slot or position was out of range
constexpr uint32_t kStatusPartials = 2;  // a merge stopped waiting for a partial

template <int D>
struct AttnShape {
  static constexpr int kTiles = D <= 128 ? 4 : 2;          // tiles per wave
  static constexpr int kSpan = kWavesA * kTiles * kTileT;  // tokens per workgroup
  static constexpr int kSteps = D / 32;                    // score MFMAs per tile
  static constexpr int kJ = D / 16;                        // output column blocks
  static constexpr int kRow = D + 4;                       // partial floats per query: D outputs, max, sum, 2 pad
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
  uint64_t* seen;
  uint32_t* counters;  // [rows * hkv * qblocks] spans done this launch
  float* partials;     // [rows * hkv * qblocks][splits][kGroupQ][kRow]
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

// p = hi + lo in the cache dtype (16-bit words).  bf16: hi is p cut to its
// top 16 bits (exact), lo the remainder p - hi (exact in fp32) cut the same
// way, so |p - hi - lo| < 2^-14 |p|.  fp16: hi is p rounded to fp16, lo the
// fp16 rounding of p - hi.
template <int DT>
__device__ __forceinline__ void split_prob(float p, uint32_t& hi, uint32_t& lo) {
  if constexpr (DT == DS_BF16) {
    const uint32_t bits = __float_as_uint(p);
    const float h = __uint_as_float(bits & 0xffff0000u);
    hi = bits >> 16;
    lo = __float_as_uint(p - h) >> 16;
  } else {
    const _Float16 h = static_cast<_Float16>(p);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(p - static_cast<float>(h)));
  }
}

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

// 16-byte accesses with the device-scope cache policy (sc1), through a raw
// buffer resource over one row's partials.
typedef __amdgpu_buffer_rsrc_t Rsrc16;
constexpr int kPolicySc1 = 16;
__device__ __forceinline__ Rsrc16 make_rsrc16(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void store16_sc1(Rsrc16 r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, static_cast<int>(off), 0, kPolicySc1);
}
__device__ __forceinline__ f32x4 load16_sc1(Rsrc16 r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, kPolicySc1));
}

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

// Run by the grid's last workgroup at its end: once every workgroup of the
// pending rows has stored its seen word (all of them have lower indices and
// were dispatched before this one), each row's working length becomes
// position + 1 and the epoch advances.
__device__ __forceinline__ void publish(const AttnArgs& a, uint32_t tag) {
  bool expired = false;
  const int seen_words = a.rows * a.hkv * a.qblocks * a.splits;
  for (int b = threadIdx.x; b < seen_words; b += kThreadsA) {
    if (b != static_cast<int>(blockIdx.x)) settle(a, a.seen + b, coherent_load(a.seen + b), tag, expired);
  }
  lds_barrier();
  for (int r = threadIdx.x; r < a.rows; r += kThreadsA) {
    const int slot = a.slots[r];
    int pos = -1;
    if (slot >= 0 && slot < a.num_slots) pos = a.positions ? a.positions[r] : a.working_lens[slot];
    if (pos >= 0 && pos < a.budget) a.working_lens[slot] = pos + 1;
    else raise_status(a, kStatusPosition);
  }
  if (threadIdx.x == 0 && a.rows > 0) coherent_store(a.header + kHdrEpoch, tag);
}

template <int DT, int D>
__global__ __launch_bounds__(kThreadsA, 2) void draft_attention_kernel(AttnArgs a) {
  using S = AttnShape<D>;
  constexpr int J = S::kJ;
  __shared__ float s_m[kWavesA][kGroupQ];
  __shared__ float s_l[kWavesA][kGroupQ];
  __shared__ float s_acc[kWavesA][kGroupQ][D + 4];
  __shared__ int s_last;
  __shared__ int s_pos;
  __shared__ uint32_t s_tag;

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

  // Thread 0 reads the launch epoch (tag = epoch + 1) and, for a pending
  // row, the row's position (scalar loads), then stores this workgroup's
  // tagged "seen" word.  The grid's last workgroup waits for every seen word
  // before it advances working_lens and the epoch, so no workgroup reads
  // either after they change.  No atomics: every word has one writer.
  const bool real = row < a.rows;
  const int slot = real ? scalar_load(a.slots + row) : -1;
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  if (threadIdx.x == 0) {
    const uint32_t epoch = static_cast<uint32_t>(scalar_load(reinterpret_cast<const int32_t*>(a.header + kHdrEpoch)));
    int pos = -1;
    if (real && slot_ok) pos = a.positions ? scalar_load(a.positions + row) : scalar_load(a.working_lens + slot);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    s_pos = (pos >= 0 && pos < a.budget) ? pos : -1;
    s_tag = epoch + 1;
    if (real) coherent_store(a.seen + blockIdx.x, tagged(epoch + 1, 0.f));
  }

  const int64_t work_base = (static_cast<int64_t>(slot_ok ? slot : 0) * a.hkv + kvh) * a.budget * D;
  const uint16_t* kw = static_cast<const uint16_t*>(a.work_k) + work_base;
  const uint16_t* vw = static_cast<const uint16_t*>(a.work_v) + work_base;
  const uint16_t* kin = static_cast<const uint16_t*>(a.k_in) + row * a.k_row + kvh * a.k_head;
  const uint16_t* vin = static_cast<const uint16_t*>(a.v_in) + row * a.v_row + kvh * a.v_head;
  const int t0 = split * S::kSpan + wave * S::kTiles * kTileT;

  // One tile's operands: K rows for the score MFMAs, V rows for the output.
  struct Tile {
    u32x4 k[S::kSteps];
    uint32_t v[4][J / 2];
  };
  // Loads of tile tb from the working rows only (rows clamped to the
  // cache); the rows from the position on are fixed up once it is known.
  auto load_tile_rows = [&](Tile& T, int tb) {
    const uint16_t* pk = kw + static_cast<int64_t>(min(tb + col, a.budget - 1)) * D + 8 * quad;
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) T.k[i] = load16(pk + 32 * i);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      load_words<J>(vw + static_cast<int64_t>(min(tb + 4 * quad + r, a.budget - 1)) * D + J * col, T.v[r]);
    }
  };
  // The first pair of the wave's tiles and this row's input K / V slices are
  // requested before the position arrives (the position is a second
  // dependent load after the slot).  Every address is valid whatever the
  // position: working rows below the cache capacity and the input row.
  Tile ta, tb_, tc, td;
  u32x4 kin_s[S::kSteps];
  uint32_t vin_s[J / 2];
  const bool early = real && slot_ok && t0 < a.budget;
  if (early) {
    load_tile_rows(ta, t0);
    load_tile_rows(tb_, t0 + kTileT);
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) kin_s[i] = load16(kin + 8 * quad + 32 * i);
    load_words<J>(vin + J * col, vin_s);
  }
  lds_barrier();
  const int pos = s_pos;
  const uint32_t tag = s_tag;
  const bool valid = pos >= 0;
  const int n = valid ? pos + 1 : 0;
  const int active = valid ? (n + S::kSpan - 1) / S::kSpan : 1;
  auto finish = [&]() {
    if (blockIdx.x == gridDim.x - 1) publish(a, tag);
  };

  if (!real) {  // padding row: zero once
    if (split == 0) zero_heads<D>(a, row, head0, gcount);
    finish();
    return;
  }
  if (split >= active) {
    finish();
    return;
  }
  if (!valid) {  // bad slot or position: zero output, touch nothing else
    zero_heads<D>(a, row, head0, gcount);
    finish();
    return;
  }

  // Query block as the B operand of the score MFMAs: lane (quad, col) holds
  // q[head0 + col][32 i + 8 quad .. + 8]; columns past the group are zero.
  // Every load of the main loop is unconditional (addresses clamped to valid
  // rows, results masked by value), so the compiler can keep the next tile's
  // loads in flight while the current tile is computed.
  u32x4 qv[S::kSteps];
  {
    const int qcol = min(col, gcount - 1);
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + row * a.q_row + (head0 + qcol) * a.q_head + 8 * quad;
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) {
      const u32x4 v = load16(qp + 32 * i);
      qv[i] = col < gcount ? v : u32x4{0, 0, 0, 0};
    }
  }

  f32x4 acc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;
  const float c = a.scale * kLog2e;

  // Rows at or past n read row n - 1 = pos (the new token's input row): a
  // valid, finite row whose scores are masked to -inf below.
  auto row_ptr = [&](const uint16_t* work, const uint16_t* in, int t) {
    return t >= pos ? in : work + static_cast<int64_t>(t) * D;
  };
  auto load_tile = [&](Tile& T, int tb) {
    const uint16_t* pk = row_ptr(kw, kin, tb + col) + 8 * quad;
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) T.k[i] = load16(pk + 32 * i);
#pragma unroll
    for (int r = 0; r < 4; ++r) load_words<J>(row_ptr(vw, vin, tb + 4 * quad + r) + J * col, T.v[r]);
  };
  // A tile loaded from the working rows: the position's row becomes the
  // input row, later rows of V become zeros (their probabilities are 0, and
  // stale cache words may not be finite; K rows there only feed masked
  // scores).
  auto fix_tile = [&](Tile& T, int tb) {
    if (tb + col == pos) {
#pragma unroll
      for (int i = 0; i < S::kSteps; ++i) T.k[i] = kin_s[i];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tb + 4 * quad + r;
#pragma unroll
      for (int w = 0; w < J / 2; ++w) T.v[r][w] = t == pos ? vin_s[w] : (t > pos ? 0u : T.v[r][w]);
    }
  };
  // Scores, online softmax and output for the 32 tokens tb .. tb + 31 held in
  // tiles T0 and T1.  The output MFMAs are 16x16x32 in the cache dtype with
  // A = V^T and B = P^T: k-slot (lane / 16, e) is token 4 * (lane / 16) +
  // (e & 3) of tile e / 4, i.e. the rows of the lane's own score tiles, and
  // head_dim column m of block j is d = J * m + j, so both operands are in the
  // lane's registers.  P is split into an upper part (its fp32 value cut to
  // the dtype) and the dtype rounding of the exact remainder; two MFMAs per
  // block keep the products within ~2^-16 of fp32 probabilities.
  auto compute_pair = [&](const Tile& T0, const Tile& T1, int tb) {
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < S::kSteps; ++i) {
      s0 = mfma_scores<DT>(T0.k[i], qv[i], s0);
      s1 = mfma_scores<DT>(T1.k[i], qv[i], s1);
    }
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = (tb + 4 * quad + i < n) ? s0[i] * c : -INFINITY;
      x[4 + i] = (tb + kTileT + 4 * quad + i < n) ? s1[i] * c : -INFINITY;
    }
    float tmax = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mn = fmaxf(m, tmax);
    const float alpha = fast_exp2(m - mn);
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = fast_exp2(x[e] - mn);
    lsum = lsum * alpha + (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
    m = mn;
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] *= alpha;
    u32x4 phi, plo;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t h0, h1, l0, l1;
      split_prob<DT>(p[2 * w], h0, l0);
      split_prob<DT>(p[2 * w + 1], h1, l1);
      phi[w] = h0 | (h1 << 16);
      plo[w] = l0 | (l1 << 16);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;  // high or low halves
      const int w = j >> 1;
      u32x4 av;
      av[0] = __builtin_amdgcn_perm(T0.v[1][w], T0.v[0][w], sel);
      av[1] = __builtin_amdgcn_perm(T0.v[3][w], T0.v[2][w], sel);
      av[2] = __builtin_amdgcn_perm(T1.v[1][w], T1.v[0][w], sel);
      av[3] = __builtin_amdgcn_perm(T1.v[3][w], T1.v[2][w], sel);
      acc[j] = mfma_scores<DT>(av, phi, acc[j]);
      acc[j] = mfma_scores<DT>(av, plo, acc[j]);
    }
  };

  // The first pair came from the working rows and is fixed up here; the
  // second pair is requested now, before the first is computed (the
  // scheduling barrier keeps the compiler from sinking the loads next to
  // their use); a pair wholly past n is loaded (cache hits on row pos) but
  // not computed.
  if (t0 < n) {
    fix_tile(ta, t0);
    fix_tile(tb_, t0 + kTileT);
    if constexpr (S::kTiles == 4) {
      load_tile(tc, t0 + 2 * kTileT);
      load_tile(td, t0 + 3 * kTileT);
      __builtin_amdgcn_sched_barrier(0);
      compute_pair(ta, tb_, t0);
      if (t0 + 2 * kTileT < n) compute_pair(tc, td, t0 + 2 * kTileT);
    } else {
      compute_pair(ta, tb_, t0);
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // The new token goes into the working cache (a workgroup of this launch
  // that reads that row of the cache early replaces it with the input row).
  if (qb == 0 && split == pos / S::kSpan && threadIdx.x < D / 4) {
    const int e = threadIdx.x % (D / 8);
    const bool is_v = threadIdx.x >= D / 8;
    uint16_t* dst = static_cast<uint16_t*>(is_v ? a.work_v : a.work_k) + work_base + static_cast<int64_t>(pos) * D;
    *reinterpret_cast<u32x4*>(dst + 8 * e) = load16((is_v ? vin : kin) + 8 * e);
  }

  // The four waves' running max, sum and unnormalised outputs go to LDS as
  // they are; one barrier, then thread t merges item (query g, outputs e ..
  // e + 3) over the waves in wave order: common max, rescaled sums.
  const int d0 = 4 * J * quad;  // lane's outputs: d = d0 + J * i + j
  if (quad == 0) {
    s_m[wave][col] = m;
    s_l[wave][col] = lsum;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < J; ++j) s_acc[wave][col][d0 + J * i + j] = acc[j][i];
  }
  lds_barrier();
  constexpr int kChunks = D / 4;
  const int items = gcount * kChunks;
  // This span's (max, sum, outputs e .. e + 3) of query g.
  auto span_item = [&](int g, int e, float& mx, float& total_l) -> f32x4 {
    mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWavesA; ++w) mx = fmaxf(mx, s_m[w][g]);
    total_l = 0.f;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWavesA; ++w) {
      const float f = fast_exp2(s_m[w][g] - mx);
      total_l += s_l[w][g] * f;
      const f32x4 x = *reinterpret_cast<const f32x4*>(&s_acc[w][g][e]);
      v = w == 0 ? x * f : v + x * f;
    }
    return v;
  };
  auto store_out = [&](int g, int e, f32x4 v, float inv) {
    uint16_t* o = static_cast<uint16_t*>(a.out) + row * a.o_row + (head0 + g) * a.o_head + e;
    const uint32_t w0 = static_cast<uint32_t>(Elem<DT>::store(v[0] * inv)) |
                        (static_cast<uint32_t>(Elem<DT>::store(v[1] * inv)) << 16);
    const uint32_t w1 = static_cast<uint32_t>(Elem<DT>::store(v[2] * inv)) |
                        (static_cast<uint32_t>(Elem<DT>::store(v[3] * inv)) << 16);
    *reinterpret_cast<u32x2*>(o) = u32x2{w0, w1};
  };

  if (active == 1) {
    for (int item = threadIdx.x; item < items; item += kThreadsA) {
      const int g = item / kChunks, e = 4 * (item % kChunks);
      float mx, total_l;
      const f32x4 v = span_item(g, e, mx, total_l);
      store_out(g, e, v, 1.f / total_l);
    }
    finish();
    return;
  }

  // Several spans.  Every span writes its result ((running max, sum,
  // unnormalised output) per query, fp32) to its slot of the row's partials
  // with device-scope stores, waits until they are done and counts itself on
  // the row's counter.  The workgroup that counts last merges the row: the
  // others' stores are complete before their counts, so it reads them
  // without waiting, and it resets the counter for the next launch.  The
  // spans are merged in index order whichever workgroup merges, so the
  // result does not depend on arrival order.
  const int unit = (row * a.hkv + kvh) * a.qblocks + qb;
  float* part_base = a.partials + static_cast<int64_t>(unit) * a.splits * kGroupQ * S::kRow;
  // The row's partials as a buffer resource: 16-byte device-scope (sc1)
  // accesses, written through to memory and read past the per-XCD caches.
  const Rsrc16 prs = make_rsrc16(part_base, static_cast<int64_t>(a.splits) * kGroupQ * S::kRow * 4);
  // Row g of a span's partial: D outputs, then (max, sum, 0, 0).
  const uint32_t span_off = static_cast<uint32_t>(split * kGroupQ * S::kRow * 4);
  for (int item = threadIdx.x; item < items; item += kThreadsA) {
    const int g = item / kChunks, e = 4 * (item % kChunks);
    float mx, total_l;
    const f32x4 v = span_item(g, e, mx, total_l);
    store16_sc1(prs, span_off + static_cast<uint32_t>((g * S::kRow + e) * 4), v);
    if (e == 0) store16_sc1(prs, span_off + static_cast<uint32_t>((g * S::kRow + D) * 4), f32x4{mx, total_l, 0.f, 0.f});
  }
  // The stores are device-scope write-throughs: once this thread's are
  // acknowledged they are visible to every workgroup.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(a.counters + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == static_cast<uint32_t>(active - 1) ? 1 : 0;
    if (s_last) coherent_store(a.counters + unit, 0u);
  }
  lds_barrier();
  if (!s_last) {
    finish();
    return;
  }

  // Merge: spans in index order, every other span's words requested at once
  // (kGroupS spans per round); this span's values come from LDS.
  for (int item = threadIdx.x; item < items; item += kThreadsA) {
    const int g = item / kChunks;
    const int e = 4 * (item % kChunks);
    float run_m = -INFINITY, run_l = 0.f;
    f32x4 run = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < active; s0 += kGroupS) {
      const int cnt = min(kGroupS, active - s0);
      f32x4 pv[kGroupS], pml[kGroupS];
#pragma unroll
      for (int u = 0; u < kGroupS; ++u) {
        const int sp = s0 + u;
        if (u < cnt && sp != split) {
          const uint32_t row_off = static_cast<uint32_t>((sp * kGroupQ + g) * S::kRow * 4);
          pv[u] = load16_sc1(prs, row_off + e * 4);
          pml[u] = load16_sc1(prs, row_off + D * 4);
        }
      }
#pragma unroll
      for (int u = 0; u < kGroupS; ++u) {
        const int sp = s0 + u;
        if (u >= cnt) break;
        float m_s, l_s;
        f32x4 a_s;
        if (sp == split) {
          a_s = span_item(g, e, m_s, l_s);
        } else {
          m_s = pml[u][0];
          l_s = pml[u][1];
          a_s = pv[u];
        }
        const float gm = fmaxf(run_m, m_s);
        const float r1 = fast_exp2(run_m - gm);
        const float r2 = fast_exp2(m_s - gm);
        run_l = run_l * r1 + l_s * r2;
        run = run * r1 + a_s * r2;
        run_m = gm;
      }
    }
    store_out(g, e, run, 1.f / run_l);
  }
  finish();
}

template <int DT, int D>
int launch_attention(hipStream_t stream, const AttnArgs& a) {
  const int64_t grid = static_cast<int64_t>(a.out_rows) * a.hkv * a.qblocks * a.splits;
  draft_attention_kernel<DT, D><<<static_cast<unsigned>(grid), kThreadsA, 0, stream>>>(a);
  return check_launch("ds_draft_attention");
}

int span_for(int head_dim) { return head_dim <= 128 ? kWavesA * 4 * kTileT : kWavesA * 2 * kTileT; }

size_t seen_bytes(size_t wgs) { return (wgs * sizeof(uint64_t) + 255) / 256 * 256; }

size_t attention_workspace_bytes(int rows, int num_q_heads, int num_kv_heads, int head_dim, int token_budget) {
  if (rows <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || token_budget <= 0) return 0;
  if (num_q_heads % num_kv_heads) return 0;
  const int group = num_q_heads / num_kv_heads;
  const int qblocks = (group + kGroupQ - 1) / kGroupQ;
  const int splits = (token_budget + span_for(head_dim) - 1) / span_for(head_dim);
  const size_t units = static_cast<size_t>(rows) * num_kv_heads * qblocks;
  const size_t wgs = units * splits;
  return kHeaderBytes + kCounterBytes + seen_bytes(wgs) + wgs * kGroupQ * (head_dim + 4) * sizeof(float);
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
  DS_SUPPORTED(static_cast<int64_t>(out_rows) * num_kv_heads * qblocks <= kMaxUnits,
               "at most %d (row, KV head, 16-query block) units per launch", kMaxUnits);
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
  const size_t units = static_cast<size_t>(rows) * num_kv_heads * qblocks;
  a.counters = reinterpret_cast<uint32_t*>(ws + kHeaderBytes);
  a.seen = reinterpret_cast<uint64_t*>(ws + kHeaderBytes + kCounterBytes);
  a.partials = reinterpret_cast<float*>(ws + kHeaderBytes + kCounterBytes + seen_bytes(units * a.splits));

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
