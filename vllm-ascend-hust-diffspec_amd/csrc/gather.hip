// Gather of selected pre-RoPE KV by plan rows, RoPE at compact local
// positions, and working-cache write — one ragged launch over all rows.
//
// Counterpart of diffspec/compact_kv.py:8-133 (kernel) and :184-242 (entry).
// Work list: each (row, block of kTileP local positions) is a tile; tiles of
// all rows are numbered through an exclusive prefix sum of per-row tile
// counts that every workgroup builds in LDS from the plan's history_len
// column, so short rows cost nothing and one launch covers a ragged batch.
// Inside a tile, lanes_per_row lanes own one (position, head) row of D
// elements; each lane moves exactly two 16-byte K vectors and two 16-byte V
// vectors, and for neox rotates its pair (x[i], x[i + rot/2]) in registers.
#include "ds355_common.h"

namespace ds355 {
namespace {

constexpr int kTileP = 32;     // local positions per tile
constexpr int kThreads = 256;  // 4 waves
constexpr int kUnroll = 4;     // (position, head) rows in flight per lane

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

__device__ __forceinline__ int row_tiles(const GatherArgs& a, int r) {
  if (a.row_active != nullptr && a.row_active[r] == 0) return 0;
  const RowPlan rp = load_row(a, r);
  return rp.len > 0 ? static_cast<int>((rp.len + kTileP - 1) / kTileP) : 0;
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

// 16-byte and 8-byte vectors carried as 32-bit words.
struct alignas(16) W4 {
  uint32_t w[4];
};
struct alignas(8) W2 {
  uint32_t w[2];
};

// Element e of a word vector, widened to fp32 (16-bit types pack two per word).
template <int DT, typename W>
__device__ __forceinline__ float elem(const W& v, int e) {
  if constexpr (sizeof(typename Elem<DT>::T) == 2) {
    return Elem<DT>::load(static_cast<uint16_t>(v.w[e >> 1] >> ((e & 1) * 16)));
  } else {
    return __uint_as_float(v.w[e]);
  }
}

// Word vector from fp32 values, each rounded to the element type.
template <int DT, typename W, int N>
__device__ __forceinline__ W pack(const float (&f)[N]) {
  W out;
  if constexpr (sizeof(typename Elem<DT>::T) == 2) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      out.w[j] = static_cast<uint32_t>(Elem<DT>::store(f[2 * j])) |
                 (static_cast<uint32_t>(Elem<DT>::store(f[2 * j + 1])) << 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out.w[j] = __float_as_uint(f[j]);
  }
  return out;
}

// Vectorised path: every lane moves 2 K + 2 V 16-byte vectors per row.
//   neox : lanes [0, half/V) rotate the pair (jV, half + jV); the other lanes
//          copy K vectors rot + (2(j - half/V) + {0,1}) V.
//   gptj : lane j handles vectors jV and D/2 + jV, each rotated in place
//          when below rot, copied otherwise.
//   V    : lane j copies vectors jV and D/2 + jV.
template <int DT, bool NEOX>
__global__ __launch_bounds__(kThreads) void gather_vec_kernel(GatherArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int V = 16 / sizeof(T);
  __shared__ int s_prefix[kMaxRows + 1];
  __shared__ int s_scratch[4];

  build_row_prefix(a.rows, s_prefix, s_scratch, [&](int r) { return row_tiles(a, r); });
  const int total = s_prefix[a.rows];

  const int D = a.head_dim;
  const int H = a.heads;
  const int half = a.rot / 2;
  const int lpr = a.lanes_per_row;
  const int rows_per_pass = kThreads / lpr;
  const int lane = static_cast<int>(threadIdx.x) % lpr;
  const int row_slot = static_cast<int>(threadIdx.x) / lpr;
  if (row_slot >= rows_per_pass) return;  // idle tail lanes when lpr does not divide 256
  const int items = kTileP * H;

  // Per-lane K job (fixed for the whole launch).
  int k_off0, k_off1;      // element offsets of the two K vectors
  bool rot0, rot1;         // gptj: rotate vector in place; neox: lane owns a pair
  int cs_off0 = 0, cs_off1 = 0;
  if (NEOX) {
    const int pairs = half / V;
    if (lane < pairs) {
      k_off0 = lane * V;
      k_off1 = half + lane * V;
      rot0 = rot1 = true;
      cs_off0 = lane * V;
    } else {
      k_off0 = a.rot + (2 * (lane - pairs)) * V;
      k_off1 = k_off0 + V;
      rot0 = rot1 = false;
    }
  } else {
    k_off0 = lane * V;
    k_off1 = D / 2 + lane * V;
    rot0 = k_off0 < a.rot;
    rot1 = k_off1 < a.rot;
    cs_off0 = k_off0 / 2;
    cs_off1 = k_off1 / 2;
  }
  const int v_off0 = lane * V;
  const int v_off1 = D / 2 + lane * V;

  const T* __restrict__ raw_k = static_cast<const T*>(a.raw_k);
  const T* __restrict__ raw_v = static_cast<const T*>(a.raw_v);
  T* __restrict__ work_k = static_cast<T*>(a.work_k);
  T* __restrict__ work_v = static_cast<T*>(a.work_v);
  const T* __restrict__ cos_sin = static_cast<const T*>(a.cos_sin);

  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const int r = find_row(s_prefix, a.rows, tile);
    const RowPlan rp = load_row(a, r);
    const int64_t p0 = static_cast<int64_t>(tile - s_prefix[r]) * kTileP;

    for (int base = row_slot; base < items; base += rows_per_pass * kUnroll) {
      W4 k0[kUnroll], k1[kUnroll], v0[kUnroll], v1[kUnroll];
      W4 c16[kUnroll], s16[kUnroll];
      W2 c8a[kUnroll], s8a[kUnroll], c8b[kUnroll], s8b[kUnroll];
      int64_t dst[kUnroll];
      // Load phase: every row of the unrolled group issues its loads first.
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int item = base + u * rows_per_pass;
        const int h = item / kTileP;
        const int64_t p = p0 + item % kTileP;
        const int64_t ap = (item < items && p < rp.len) ? abs_position(a, r, rp, p) : -1;
        dst[u] = ap >= 0 ? ((rp.slot * H + h) * static_cast<int64_t>(a.budget) + p) * D : -1;
        k0[u] = k1[u] = v0[u] = v1[u] = c16[u] = s16[u] = W4{{0u, 0u, 0u, 0u}};
        c8a[u] = s8a[u] = c8b[u] = s8b[u] = W2{{0u, 0u}};
        if (ap >= 0) {
          const int64_t src = ((rp.slot * a.max_model_len + ap) * H + h) * static_cast<int64_t>(D);
          k0[u] = *reinterpret_cast<const W4*>(raw_k + src + k_off0);
          k1[u] = *reinterpret_cast<const W4*>(raw_k + src + k_off1);
          v0[u] = *reinterpret_cast<const W4*>(raw_v + src + v_off0);
          v1[u] = *reinterpret_cast<const W4*>(raw_v + src + v_off1);
          const T* cs_row = cos_sin + p * a.cs_stride;
          if (NEOX) {
            if (rot0) {
              c16[u] = *reinterpret_cast<const W4*>(cs_row + cs_off0);
              s16[u] = *reinterpret_cast<const W4*>(cs_row + half + cs_off0);
            }
          } else {
            if (rot0) {
              c8a[u] = *reinterpret_cast<const W2*>(cs_row + cs_off0);
              s8a[u] = *reinterpret_cast<const W2*>(cs_row + half + cs_off0);
            }
            if (rot1) {
              c8b[u] = *reinterpret_cast<const W2*>(cs_row + cs_off1);
              s8b[u] = *reinterpret_cast<const W2*>(cs_row + half + cs_off1);
            }
          }
        }
      }
      // Rotate + store phase.
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (dst[u] >= 0) {
          W4 ok0 = k0[u], ok1 = k1[u];
          if (NEOX) {
            if (rot0) {
              float f1[V], f2[V];
#pragma unroll
              for (int e = 0; e < V; ++e) {
                rotate_pair(elem<DT>(k0[u], e), elem<DT>(k1[u], e), elem<DT>(c16[u], e), elem<DT>(s16[u], e),
                            f1[e], f2[e]);
              }
              ok0 = pack<DT, W4>(f1);
              ok1 = pack<DT, W4>(f2);
            }
          } else {
            if (rot0) {
              float f[V];
#pragma unroll
              for (int e = 0; e < V / 2; ++e) {
                rotate_pair(elem<DT>(k0[u], 2 * e), elem<DT>(k0[u], 2 * e + 1), elem<DT>(c8a[u], e),
                            elem<DT>(s8a[u], e), f[2 * e], f[2 * e + 1]);
              }
              ok0 = pack<DT, W4>(f);
            }
            if (rot1) {
              float f[V];
#pragma unroll
              for (int e = 0; e < V / 2; ++e) {
                rotate_pair(elem<DT>(k1[u], 2 * e), elem<DT>(k1[u], 2 * e + 1), elem<DT>(c8b[u], e),
                            elem<DT>(s8b[u], e), f[2 * e], f[2 * e + 1]);
              }
              ok1 = pack<DT, W4>(f);
            }
          }
          *reinterpret_cast<W4*>(work_k + dst[u] + k_off0) = ok0;
          *reinterpret_cast<W4*>(work_k + dst[u] + k_off1) = ok1;
          *reinterpret_cast<W4*>(work_v + dst[u] + v_off0) = v0[u];
          *reinterpret_cast<W4*>(work_v + dst[u] + v_off1) = v1[u];
        }
      }
    }
  }
}

// General path for shapes the vector path does not cover (head_dim or the
// rotary split not a multiple of the 16-byte vector): one thread per
// (position, head) row, element by element.
template <int DT>
__global__ __launch_bounds__(kThreads) void gather_scalar_kernel(GatherArgs a, int neox) {
  using E = Elem<DT>;
  using T = typename E::T;
  __shared__ int s_prefix[kMaxRows + 1];
  __shared__ int s_scratch[4];
  build_row_prefix(a.rows, s_prefix, s_scratch, [&](int r) { return row_tiles(a, r); });
  const int total = s_prefix[a.rows];
  const int D = a.head_dim;
  const int H = a.heads;
  const int half = a.rot / 2;
  const T* raw_k = static_cast<const T*>(a.raw_k);
  const T* raw_v = static_cast<const T*>(a.raw_v);
  T* work_k = static_cast<T*>(a.work_k);
  T* work_v = static_cast<T*>(a.work_v);
  const T* cos_sin = static_cast<const T*>(a.cos_sin);
  const int items = kTileP * H;
  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const int r = find_row(s_prefix, a.rows, tile);
    const RowPlan rp = load_row(a, r);
    const int64_t p0 = static_cast<int64_t>(tile - s_prefix[r]) * kTileP;
    for (int item = threadIdx.x; item < items; item += kThreads) {
      const int h = item / kTileP;
      const int64_t p = p0 + item % kTileP;
      if (p >= rp.len) continue;
      const int64_t ap = abs_position(a, r, rp, p);
      if (ap < 0) continue;
      const int64_t src = ((rp.slot * a.max_model_len + ap) * H + h) * static_cast<int64_t>(D);
      const int64_t dst = ((rp.slot * H + h) * static_cast<int64_t>(a.budget) + p) * D;
      const T* cs_row = cos_sin + p * a.cs_stride;
      for (int i = 0; i < half; ++i) {
        const int i1 = neox ? i : 2 * i;
        const int i2 = neox ? i + half : 2 * i + 1;
        float o1, o2;
        rotate_pair(E::load(raw_k[src + i1]), E::load(raw_k[src + i2]), E::load(cs_row[i]),
                    E::load(cs_row[half + i]), o1, o2);
        work_k[dst + i1] = E::store(o1);
        work_k[dst + i2] = E::store(o2);
      }
      for (int d = a.rot; d < D; ++d) work_k[dst + d] = raw_k[src + d];
      for (int d = 0; d < D; ++d) work_v[dst + d] = raw_v[src + d];
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT>
int launch_gather(hipStream_t stream, GatherArgs a, bool neox, int grid) {
  using T = typename Elem<DT>::T;
  constexpr int V = 16 / sizeof(T);
  const int D = a.head_dim;
  bool vec = (D % (2 * V) == 0) && aligned16(a.raw_k) && aligned16(a.raw_v) && aligned16(a.work_k) &&
             aligned16(a.work_v) && (D / (2 * V)) <= kThreads;
  if (a.rot > 0) {
    vec = vec && (a.cs_stride % V == 0) && aligned16(a.cos_sin);
    if (neox) vec = vec && ((a.rot / 2) % V == 0);
    else vec = vec && (a.rot % V == 0);
  }
  if (vec) {
    a.lanes_per_row = D / (2 * V);
    if (neox) gather_vec_kernel<DT, true><<<grid, kThreads, 0, stream>>>(a);
    else gather_vec_kernel<DT, false><<<grid, kThreads, 0, stream>>>(a);
  } else {
    a.lanes_per_row = 1;
    gather_scalar_kernel<DT><<<grid, kThreads, 0, stream>>>(a, neox ? 1 : 0);
  }
  return check_launch("ds_rebuild_compact_kv");
}

}  // namespace

int rebuild_compact_kv_impl(hipStream_t stream, int dtype, const void* raw_key, const void* raw_value,
                            void* working_key, void* working_value, const int64_t* plan, int rows,
                            int plan_width, const void* cos_sin, int64_t cs_stride, int cs_rows, int num_slots,
                            int max_model_len, int heads, int head_dim, int token_budget, int chunk_size,
                            int rotary_dim, int is_neox_style, int max_width, const int32_t* row_active,
                            bool padded_rows) {
  DS_REQUIRE(dtype == DS_BF16 || dtype == DS_FP16 || dtype == DS_FP32, "KV caches must use BF16, FP16 or FP32");
  DS_REQUIRE(rows >= 0 && num_slots > 0 && max_model_len > 0 && heads > 0 && head_dim > 0,
             "raw sequence, head and head dimensions must be positive");
  // Plans of a padded batch may have more rows than slots (padding rows are empty).
  DS_REQUIRE(padded_rows || rows <= num_slots, "KV plan exceeds the working cache batch or token capacity");
  DS_REQUIRE(max_width >= 0 && max_width <= token_budget,
             "KV plan exceeds the working cache batch or token capacity");
  DS_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0,
             "rotary_dim must be even and between zero and head_dim");
  DS_REQUIRE(chunk_size > 0 && plan_width == 5 + token_budget / chunk_size,
             "plan width must be 5 + working_budget // chunk_size");
  DS_REQUIRE(cs_rows >= max_width && cs_stride >= rotary_dim, "cos/sin cache must contain all local positions and rotary dimensions");
  DS_SUPPORTED(rows <= kMaxRows, "at most %d plan rows per launch (got %d)", kMaxRows, rows);
  if (rows == 0 || max_width == 0) return clear_error();
  DS_REQUIRE(raw_key && raw_value && working_key && working_value && plan, "null tensor pointer");
  DS_REQUIRE(rotary_dim == 0 || cos_sin, "null cos/sin pointer");

  GatherArgs a{};
  a.raw_k = raw_key;
  a.raw_v = raw_value;
  a.work_k = working_key;
  a.work_v = working_value;
  a.plan = plan;
  a.row_active = row_active;
  a.cos_sin = cos_sin;
  a.cs_stride = cs_stride;
  a.rows = rows;
  a.plan_width = plan_width;
  a.num_slots = num_slots;
  a.max_model_len = max_model_len;
  a.heads = heads;
  a.head_dim = head_dim;
  a.budget = token_budget;
  a.chunk = chunk_size;
  a.rot = rotary_dim;
  int limit = (max_width + 15) / 16 * 16;  // the reference's 16-token grid
  if (limit > token_budget) limit = token_budget;
  if (rotary_dim > 0 && limit > cs_rows) limit = cs_rows;
  a.pos_limit = limit;

  const int tiles_per_row = (limit + kTileP - 1) / kTileP;
  const int64_t max_tiles = static_cast<int64_t>(rows) * tiles_per_row;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 8;
  const int grid = static_cast<int>(max_tiles < cap ? max_tiles : cap);
  if (grid <= 0) return clear_error();
  const bool neox = is_neox_style != 0;
  switch (dtype) {
    case DS_BF16: return launch_gather<DS_BF16>(stream, a, neox, grid);
    case DS_FP16: return launch_gather<DS_FP16>(stream, a, neox, grid);
    default: return launch_gather<DS_FP32>(stream, a, neox, grid);
  }
}

}  // namespace ds355

extern "C" int ds_rebuild_compact_kv(ds_stream_t stream, int dtype, const void* raw_key, const void* raw_value,
                                     void* working_key, void* working_value, const int64_t* plan, int rows,
                                     int plan_width, const void* cos_sin, int64_t cs_stride, int cs_rows,
                                     int num_slots, int max_model_len, int heads, int head_dim, int token_budget,
                                     int chunk_size, int rotary_dim, int is_neox_style, int max_width,
                                     const int32_t* row_active) {
  return ds355::rebuild_compact_kv_impl(reinterpret_cast<hipStream_t>(stream), dtype, raw_key, raw_value,
                                        working_key, working_value, plan, rows, plan_width, cos_sin, cs_stride,
                                        cs_rows, num_slots, max_model_len, heads, head_dim, token_budget,
                                        chunk_size, rotary_dim, is_neox_style, max_width, row_active, false);
}
