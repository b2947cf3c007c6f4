// Gather + RoPE + working-cache write of one task (ppw consecutive local
// positions of one plan row, every head), shared by gather_wave_kernel and
// the fused retrieval step.  See gather.hip for the layout.
#pragma once

#include "ds355_common.h"

namespace ds355 {
namespace gather {

constexpr int kTileP = 32;     // local positions per tile
constexpr int kThreads = 256;  // 4 waves

struct GatherArgs {
  const void* raw_k;
  const void* raw_v;
  void* work_k;
  void* work_v;
  const int64_t* plan;
  const int32_t* row_active;
  const void* cos_sin;
  int64_t cs_stride;
  int rows, plan_width, num_slots, max_model_len, heads, head_dim, budget, chunk, rot;
  int pos_limit;  // positions p >= pos_limit are never touched
  int lanes_per_row;
};

struct RowPlan {
  int64_t slot, len, tail_start, prefix_len, drop;
};

__device__ __forceinline__ RowPlan load_row(const GatherArgs& a, int r) {
  const int64_t* row = a.plan + static_cast<int64_t>(r) * a.plan_width;
  RowPlan rp;
  rp.slot = row[0];
  rp.len = row[1];
  rp.tail_start = row[2];
  rp.prefix_len = row[3];
  rp.drop = row[4];
  if (rp.len > a.pos_limit) rp.len = a.pos_limit;
  if (rp.slot < 0 || rp.slot >= a.num_slots) rp.len = 0;
  return rp;
}

// Local positions of row r that the gather moves (0 for inactive, padding
// or empty rows).
__device__ __forceinline__ int row_len(const GatherArgs& a, int r) {
  if (a.row_active != nullptr && a.row_active[r] == 0) return 0;
  const RowPlan rp = load_row(a, r);
  return rp.len > 0 ? static_cast<int>(rp.len) : 0;
}

__device__ __forceinline__ int row_tiles(const GatherArgs& a, int r) {
  return (row_len(a, r) + kTileP - 1) / kTileP;
}

// Absolute raw position of local position p (compact_kv.py:40-52); -1 when
// the plan points outside the row or the raw cache.
__device__ __forceinline__ int64_t abs_position(const GatherArgs& a, int r, const RowPlan& rp, int64_t p) {
  int64_t pos;
  if (p < rp.prefix_len) {
    const int64_t pp = p + rp.drop;
    const int64_t col = 5 + pp / a.chunk;
    if (col >= a.plan_width) return -1;
    pos = a.plan[static_cast<int64_t>(r) * a.plan_width + col] * a.chunk + pp % a.chunk;
  } else {
    pos = rp.tail_start + p - rp.prefix_len;
  }
  return (pos >= 0 && pos < a.max_model_len) ? pos : -1;
}

// Rotation of one pair in fp32 with every product and the sum rounded
// separately (no contraction), as the CPU oracle computes it.
__device__ __forceinline__ void rotate_pair(float x1, float x2, float c, float s, float& o1, float& o2) {
#pragma clang fp contract(off)
  const float a = x1 * c;
  const float b = x2 * s;
  const float d = x2 * c;
  const float e = x1 * s;
  o1 = a - b;
  o2 = d + e;
}

// The same rotation for bf16 values with one fused multiply-add per output:
// o1 = fma(x1, c, -(x2 * s)), o2 = fma(x1, s, x2 * c).  A product of two
// bf16 values has at most 16 significant bits, so it is exact in fp32
// unless it is nonzero and below fp32's smallest normal, 2^-126 (a key
// below 2^-100 against a table value below 2^-26, far from any model's
// keys).  Then x1 * c and x2 * s need no rounding, and the fma rounds the
// same exact sum once, as the oracle's subtraction does, signed zeros
// included (IEEE fma: a zero sum is -0 only when both terms are -0).
__device__ __forceinline__ void rotate_pair_bf16(float x1, float x2, float c, float s, float& o1, float& o2) {
  o1 = __builtin_fmaf(x1, c, -(x2 * s));
  o2 = __builtin_fmaf(x1, s, x2 * c);
}
// bf16 halves of a word widened to fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// Two fp32 values rounded to bf16 (round to nearest even, v_cvt_pk_bf16_f32)
// and packed lo | hi << 16; NaN becomes 0x7fc0, the oracle's rule.
typedef __bf16 BF2 __attribute__((ext_vector_type(2)));
typedef float F2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  lo = lo == lo ? lo : __uint_as_float(0x7fc00000u);
  hi = hi == hi ? hi : __uint_as_float(0x7fc00000u);
  const F2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, BF2));
}

// 16-byte and 8-byte vectors carried as 32-bit words.  Native vector types
// (not arrays in a struct) keep arrays of them in registers.
typedef uint32_t W4 __attribute__((ext_vector_type(4)));
typedef uint32_t W2 __attribute__((ext_vector_type(2)));

// Element e of a word vector, widened to fp32 (16-bit types pack two per word).
template <int DT, typename W>
__device__ __forceinline__ float elem(const W& v, int e) {
  if constexpr (sizeof(typename Elem<DT>::T) == 2) {
    return Elem<DT>::load(static_cast<uint16_t>(v[e >> 1] >> ((e & 1) * 16)));
  } else {
    return __uint_as_float(v[e]);
  }
}

// Word vector from fp32 values, each rounded to the element type.
template <int DT, typename W, int N>
__device__ __forceinline__ W pack(const float (&f)[N]) {
  W out;
  if constexpr (sizeof(typename Elem<DT>::T) == 2) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      out[j] = static_cast<uint32_t>(Elem<DT>::store(f[2 * j])) |
                 (static_cast<uint32_t>(Elem<DT>::store(f[2 * j + 1])) << 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = __float_as_uint(f[j]);
  }
  return out;
}

// Raw buffer access (CDNA buffer instructions): a 128-bit resource in SGPRs
// holds a wave-uniform base and a byte size; lanes pass 32-bit byte offsets
// and the scalar offset steps between heads.  An offset at or past the size
// reads zeros and drops stores in hardware, which masks idle lanes without
// branches.  0x00020000 is the raw (untyped) resource word of the gfx9 family.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kOutOfRange = 0x80000000u;  // beyond every resource size used here (< 2 GiB)

__device__ __forceinline__ Rsrc make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ W4 buf_load16(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}
__device__ __forceinline__ W2 buf_load8(Rsrc r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(voff), 0, 0);
}
// Working-cache rows are written once per rebuild and not read again by
// this launch: non-temporal stores (cache policy bit 1, nt) keep them from
// displacing cached lines, measured about 15% faster than cached stores when
// the gathered rows are not already in the MALL.
constexpr int kStoreNT = 2;
__device__ __forceinline__ void buf_store16(W4 v, Rsrc r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(voff), static_cast<int>(soff), kStoreNT);
}

// Per-lane constants of the vector path, computed once per wave.
struct GatherLane {
  int q;         // position within the task
  int j;         // slice of the head dimension
  bool lane_ok;  // false only for idle tail lanes when lanes_per_row does not divide 64
  int k_off0, k_off1;  // element offsets of the two K vectors
  bool rot0, rot1;     // gptj: rotate the vector in place; neox: the lane owns a pair
  int cs_off0, cs_off1;
  int v_off0, v_off1;
  int64_t raw_slot_bytes, work_slot_bytes;
  uint32_t raw_head, work_head;
  Rsrc cs;
  int ncol;  // chunk-id columns of a plan row
};

template <int DT, bool NEOX>
__device__ __forceinline__ GatherLane gather_lane(const GatherArgs& a) {
  using T = typename Elem<DT>::T;
  constexpr int V = 16 / sizeof(T);
  constexpr int SZ = sizeof(T);
  GatherLane L;
  const int lpr = a.lanes_per_row;
  const int ppw = 64 / lpr;
  const int D = a.head_dim;
  const int H = a.heads;
  const int half = a.rot / 2;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  L.q = lane / lpr;
  L.j = lane - L.q * lpr;
  L.lane_ok = L.q < ppw;
  const int j = L.j;
  L.cs_off0 = 0;
  L.cs_off1 = 0;
  if (NEOX) {
    const int pairs = half / V;
    if (j < pairs) {
      L.k_off0 = j * V;
      L.k_off1 = half + j * V;
      L.rot0 = L.rot1 = true;
      L.cs_off0 = j * V;
    } else {
      L.k_off0 = a.rot + (2 * (j - pairs)) * V;
      L.k_off1 = L.k_off0 + V;
      L.rot0 = L.rot1 = false;
    }
  } else {
    L.k_off0 = j * V;
    L.k_off1 = D / 2 + j * V;
    L.rot0 = L.k_off0 < a.rot;
    L.rot1 = L.k_off1 < a.rot;
    L.cs_off0 = L.k_off0 / 2;
    L.cs_off1 = L.k_off1 / 2;
  }
  L.v_off0 = j * V;
  L.v_off1 = D / 2 + j * V;
  L.raw_slot_bytes = static_cast<int64_t>(a.max_model_len) * H * D * SZ;
  L.work_slot_bytes = static_cast<int64_t>(H) * a.budget * D * SZ;
  L.raw_head = static_cast<uint32_t>(D * SZ);
  L.work_head = static_cast<uint32_t>(static_cast<int64_t>(a.budget) * D * SZ);
  L.cs = make_rsrc(a.cos_sin, static_cast<int64_t>(a.pos_limit) * a.cs_stride * SZ);
  L.ncol = a.plan_width - 5;
  return L;
}

// Moves local positions p0 .. p0 + ppw - 1 of one plan row (fields slot ..
// drop, wave-uniform; len already clamped to pos_limit and 0 for an invalid
// slot).  chunk_id(c) returns the plan row's chunk id column c.
template <int DT, bool NEOX, int HG, typename ChunkId>
__device__ __forceinline__ void gather_task(const GatherArgs& a, const GatherLane& L, int p0, int64_t slot,
                                            int64_t len, int64_t tail_start, int64_t prefix_len, int64_t drop,
                                            ChunkId chunk_id) {
  using T = typename Elem<DT>::T;
  constexpr int V = 16 / sizeof(T);
  constexpr int SZ = sizeof(T);
  const int D = a.head_dim;
  const int H = a.heads;
  const int half = a.rot / 2;
  const int q = L.q;
  const bool lane_ok = L.lane_ok;
  const int k_off0 = L.k_off0, k_off1 = L.k_off1, v_off0 = L.v_off0, v_off1 = L.v_off1;
  const bool rot0 = L.rot0, rot1 = L.rot1;
  const int cs_off0 = L.cs_off0, cs_off1 = L.cs_off1;
  const int64_t raw_slot_bytes = L.raw_slot_bytes, work_slot_bytes = L.work_slot_bytes;
  const uint32_t raw_head = L.raw_head, work_head = L.work_head;
  const Rsrc cs = L.cs;
  const int ncol = L.ncol;
  // Absolute raw position of local position p (compact_kv.py:40-52).
  const int64_t p = p0 + q;
  const int64_t pp = p + drop;
  const int64_t col = pp >= 0 ? pp / a.chunk : -1;
  int64_t cid = 0;
  if (ncol > 0) cid = chunk_id(min(max(col, static_cast<int64_t>(0)), static_cast<int64_t>(ncol - 1)));
  const bool in_prefix = p < prefix_len;
  const int64_t pos = in_prefix ? cid * a.chunk + (pp - col * a.chunk) : tail_start + p - prefix_len;
  const bool ok = lane_ok && p < len && (!in_prefix || (col >= 0 && col < ncol)) && pos >= 0 &&
                  pos < a.max_model_len;

  const Rsrc rk = make_rsrc(static_cast<const char*>(a.raw_k) + slot * raw_slot_bytes, raw_slot_bytes);
  const Rsrc rv = make_rsrc(static_cast<const char*>(a.raw_v) + slot * raw_slot_bytes, raw_slot_bytes);
  const Rsrc wk = make_rsrc(static_cast<const char*>(a.work_k) + slot * work_slot_bytes, work_slot_bytes);
  const Rsrc wv = make_rsrc(static_cast<const char*>(a.work_v) + slot * work_slot_bytes, work_slot_bytes);
  const uint32_t src = ok ? static_cast<uint32_t>(pos * H * D * SZ) : kOutOfRange;
  const uint32_t dst = ok ? static_cast<uint32_t>(p * D * SZ) : kOutOfRange;
  const uint32_t csr = ok ? static_cast<uint32_t>(p * a.cs_stride * SZ) : kOutOfRange;

  W4 c16 = W4{0u, 0u, 0u, 0u}, s16 = W4{0u, 0u, 0u, 0u};
  W2 c8a = W2{0u, 0u}, s8a = W2{0u, 0u}, c8b = W2{0u, 0u}, s8b = W2{0u, 0u};
  if (NEOX) {
    if (rot0) {
      c16 = buf_load16(cs, csr + cs_off0 * SZ, 0);
      s16 = buf_load16(cs, csr + (half + cs_off0) * SZ, 0);
    }
  } else {
    if (rot0) {
      c8a = buf_load8(cs, csr + cs_off0 * SZ);
      s8a = buf_load8(cs, csr + (half + cs_off0) * SZ);
    }
    if (rot1) {
      c8b = buf_load8(cs, csr + cs_off1 * SZ);
      s8b = buf_load8(cs, csr + (half + cs_off1) * SZ);
    }
  }

  for (int h0 = 0; h0 < H; h0 += HG) {
    W4 k0[HG], k1[HG], v0[HG], v1[HG];
#pragma unroll
    for (int u = 0; u < HG; ++u) {
      const uint32_t hs = static_cast<uint32_t>(min(h0 + u, H - 1)) * raw_head;
      k0[u] = buf_load16(rk, src + k_off0 * SZ, hs);
      k1[u] = buf_load16(rk, src + k_off1 * SZ, hs);
      v0[u] = buf_load16(rv, src + v_off0 * SZ, hs);
      v1[u] = buf_load16(rv, src + v_off1 * SZ, hs);
    }
#pragma unroll
    for (int u = 0; u < HG; ++u) {
      if (h0 + u >= H) break;  // wave-uniform
      W4 ok0 = k0[u], ok1 = k1[u];
      if constexpr (DT == DS_BF16) {
        if (NEOX) {
          // Word w of k0 / k1 holds x1 / x2 of elements 2w and 2w + 1.
          if (rot0) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              float a0, a1, b0, b1;
              rotate_pair_bf16(bf16_lo(k0[u][w]), bf16_lo(k1[u][w]), bf16_lo(c16[w]), bf16_lo(s16[w]), a0, b0);
              rotate_pair_bf16(bf16_hi(k0[u][w]), bf16_hi(k1[u][w]), bf16_hi(c16[w]), bf16_hi(s16[w]), a1, b1);
              ok0[w] = pack_bf16(a0, a1);
              ok1[w] = pack_bf16(b0, b1);
            }
          }
        } else {
          // Word e holds the pair (x1, x2); its cos/sin are element e of the
          // 8-byte table vectors.
          if (rot0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t c = c8a[e >> 1], sn = s8a[e >> 1];
              float o1, o2;
              rotate_pair_bf16(bf16_lo(k0[u][e]), bf16_hi(k0[u][e]), (e & 1) ? bf16_hi(c) : bf16_lo(c),
                               (e & 1) ? bf16_hi(sn) : bf16_lo(sn), o1, o2);
              ok0[e] = pack_bf16(o1, o2);
            }
          }
          if (rot1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t c = c8b[e >> 1], sn = s8b[e >> 1];
              float o1, o2;
              rotate_pair_bf16(bf16_lo(k1[u][e]), bf16_hi(k1[u][e]), (e & 1) ? bf16_hi(c) : bf16_lo(c),
                               (e & 1) ? bf16_hi(sn) : bf16_lo(sn), o1, o2);
              ok1[e] = pack_bf16(o1, o2);
            }
          }
        }
      } else if (NEOX) {
        if (rot0) {
          float f1[V], f2[V];
#pragma unroll
          for (int e = 0; e < V; ++e) {
            rotate_pair(elem<DT>(k0[u], e), elem<DT>(k1[u], e), elem<DT>(c16, e), elem<DT>(s16, e), f1[e], f2[e]);
          }
          ok0 = pack<DT, W4>(f1);
          ok1 = pack<DT, W4>(f2);
        }
      } else {
        if (rot0) {
          float f[V];
#pragma unroll
          for (int e = 0; e < V / 2; ++e) {
            rotate_pair(elem<DT>(k0[u], 2 * e), elem<DT>(k0[u], 2 * e + 1), elem<DT>(c8a, e), elem<DT>(s8a, e),
                        f[2 * e], f[2 * e + 1]);
          }
          ok0 = pack<DT, W4>(f);
        }
        if (rot1) {
          float f[V];
#pragma unroll
          for (int e = 0; e < V / 2; ++e) {
            rotate_pair(elem<DT>(k1[u], 2 * e), elem<DT>(k1[u], 2 * e + 1), elem<DT>(c8b, e), elem<DT>(s8b, e),
                        f[2 * e], f[2 * e + 1]);
          }
          ok1 = pack<DT, W4>(f);
        }
      }
      const uint32_t hd = static_cast<uint32_t>(h0 + u) * work_head;
      buf_store16(ok0, wk, dst + k_off0 * SZ, hd);
      buf_store16(ok1, wk, dst + k_off1 * SZ, hd);
      buf_store16(v0[u], wv, dst + v_off0 * SZ, hd);
      buf_store16(v1[u], wv, dst + v_off1 * SZ, hd);
    }
  }
}

// Gather records: what the working cache holds per (slot, task of ppw local
// positions), so a rebuild can leave out tasks whose bytes it would rewrite
// unchanged.
//   - A task of local positions [p0, p0 + ppw) lying wholly in the plan's
//     history prefix (p0 + ppw <= prefix_len) holds bytes that depend only
//     on the slot's chunk ids, the prefix drop and the raw rows they point
//     to: its record is (selection generation << 32) | (drop + 1), which
//     stays valid from one draft cycle to the next.
//   - Any other task wholly inside the history (p0 + ppw <= len) depends on
//     the whole plan, which is a function of the slot's selection and the
//     history end (the root position, tail_start + len - prefix_len): its
//     record is (generation << 32) | 2^31 | end, valid for that root only.
//   - A task cut by the history's end has record 0.
// Raw rows before a request's committed root are not rewritten while the
// request holds its slot (the draft only appends), the draft attention
// writes the working cache only at and past the history's end, and a slot's
// generation changes with every stored selection and every change of the
// request holding it, so an equal record means equal bytes.  drop + 1 and
// end are below 2^31, so the two kinds never meet.
__device__ __forceinline__ uint64_t history_record(int p0, int ppw, int64_t len, int64_t tail_start,
                                                   int64_t prefix_len, int64_t drop, uint32_t gen) {
  const uint64_t g = static_cast<uint64_t>(gen) << 32;
  if (p0 + ppw <= prefix_len) return g | static_cast<uint64_t>(drop + 1);
  if (p0 + ppw <= len) return g | 0x80000000u | static_cast<uint64_t>(tail_start + len - prefix_len);
  return 0u;
}

// Whether every raw row task [p0, p0 + ppw) reads lies below `first_rw`, the
// first raw position the draft's prefill of this step rewrites: prefix rows
// lie below tail_start, tail position p reads tail_start + p - prefix_len.
__device__ __forceinline__ bool sources_final(int p0, int ppw, int64_t tail_start, int64_t prefix_len,
                                              int64_t first_rw) {
  const int64_t last = p0 + ppw - 1;
  if (tail_start > first_rw) return false;
  return last < prefix_len || tail_start + (last - prefix_len) < first_rw;
}

}  // namespace gather
}  // namespace ds355
