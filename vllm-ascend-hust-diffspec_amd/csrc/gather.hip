// Gather of selected pre-RoPE KV by plan rows, RoPE at compact local
// positions, and working-cache write — one ragged launch over all rows.
//
// Counterpart of diffspec/compact_kv.py:8-133 (kernel) and :184-242 (entry).
// Work list: the positions of every row are cut into tasks of a few
// consecutive local positions; tasks of all rows are numbered through an
// exclusive prefix sum of per-row task counts that every workgroup builds in
// LDS from the plan's history_len column, so short rows cost nothing and one
// launch covers a ragged batch.  In the vector path each wave works through
// its own task list; a lane owns one position and one slice of the head
// dimension (two 16-byte K and two 16-byte V vectors per head), rotates its
// neox pairs (x[i], x[i + rot/2]) or GPT-J pairs in registers, and reuses the
// position's cos/sin for every head.
#include "ds355_common.h"

namespace ds355 {
namespace {

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

// Vectorised path.  Waves are independent workers (no block barrier after
// the prologue).  A task is (row, ppw consecutive local positions) for every
// head; ppw = 64 / lanes_per_row.  Lane l owns position p0 + l / lanes_per_row
// and slice j = l % lanes_per_row of the head dimension, where it moves two
// 16-byte K vectors and two 16-byte V vectors per head:
//   neox : slices [0, half/V) rotate the pair (jV, half + jV); the other
//          slices copy K vectors rot + (2(j - half/V) + {0,1}) V.
//   gptj : slice j handles vectors jV and D/2 + jV, each rotated in place
//          when below rot, copied otherwise.
//   V    : slice j copies vectors jV and D/2 + jV.
// The cos/sin vectors of the lane's position are loaded once and reused for
// every head.  Plan fields are wave-uniform and come through scalar loads;
// only the chunk id of a prefix position is a per-lane load.  Resources span
// one slot's raw cache ([max_model_len, H, D], below 2 GiB: checked on the
// host) and one slot's working cache ([H, budget, D]); a lane with nothing
// to move uses an out-of-range offset.  HG = heads in flight at once.
template <int DT, bool NEOX, int HG>
__global__ __launch_bounds__(kThreads) void gather_wave_kernel(GatherArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int V = 16 / sizeof(T);
  constexpr int SZ = sizeof(T);
  __shared__ int s_prefix[kMaxRows + 1];
  __shared__ int s_scratch[4];

  const int lpr = a.lanes_per_row;
  const int ppw = 64 / lpr;
  build_row_prefix(a.rows, s_prefix, s_scratch, [&](int r) { return (row_len(a, r) + ppw - 1) / ppw; });
  const int total = s_prefix[a.rows];

  const int D = a.head_dim;
  const int H = a.heads;
  const int half = a.rot / 2;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int q = lane / lpr;      // position within the task
  const int j = lane - q * lpr;  // slice of the head dimension
  const bool lane_ok = q < ppw;  // false only for idle tail lanes when lpr does not divide 64

  int k_off0, k_off1;  // element offsets of the two K vectors
  bool rot0, rot1;     // gptj: rotate the vector in place; neox: the lane owns a pair
  int cs_off0 = 0, cs_off1 = 0;
  if (NEOX) {
    const int pairs = half / V;
    if (j < pairs) {
      k_off0 = j * V;
      k_off1 = half + j * V;
      rot0 = rot1 = true;
      cs_off0 = j * V;
    } else {
      k_off0 = a.rot + (2 * (j - pairs)) * V;
      k_off1 = k_off0 + V;
      rot0 = rot1 = false;
    }
  } else {
    k_off0 = j * V;
    k_off1 = D / 2 + j * V;
    rot0 = k_off0 < a.rot;
    rot1 = k_off1 < a.rot;
    cs_off0 = k_off0 / 2;
    cs_off1 = k_off1 / 2;
  }
  const int v_off0 = j * V;
  const int v_off1 = D / 2 + j * V;

  const int64_t raw_slot_bytes = static_cast<int64_t>(a.max_model_len) * H * D * SZ;
  const int64_t work_slot_bytes = static_cast<int64_t>(H) * a.budget * D * SZ;
  const uint32_t raw_head = static_cast<uint32_t>(D * SZ);
  const uint32_t work_head = static_cast<uint32_t>(static_cast<int64_t>(a.budget) * D * SZ);
  const Rsrc cs = make_rsrc(a.cos_sin, static_cast<int64_t>(a.pos_limit) * a.cs_stride * SZ);
  const int ncol = a.plan_width - 5;  // chunk-id columns of a plan row

  const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6));
  const int tw = gridDim.x * (kThreads / 64);
  int hint = 0;
  for (int task = gw; task < total; task += tw) {
    int lo = hint, hi = a.rows - 1;  // task numbers grow along the wave's list
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_prefix[mid] <= task) lo = mid; else hi = mid - 1;
    }
    hint = lo;
    const int r = __builtin_amdgcn_readfirstlane(lo);  // uniform (LDS reads are not known to be)
    const int p0 = __builtin_amdgcn_readfirstlane((task - s_prefix[r]) * ppw);
    const int64_t* prow = a.plan + static_cast<int64_t>(r) * a.plan_width;
    const int64_t slot = scalar_load(prow + 0);
    const int64_t len = min(scalar_load(prow + 1), static_cast<int64_t>(a.pos_limit));
    const int64_t tail_start = scalar_load(prow + 2);
    const int64_t prefix_len = scalar_load(prow + 3);
    const int64_t drop = scalar_load(prow + 4);

    // Absolute raw position of local position p (compact_kv.py:40-52).
    const int64_t p = p0 + q;
    const int64_t pp = p + drop;
    const int64_t col = pp >= 0 ? pp / a.chunk : -1;
    int64_t cid = 0;
    if (ncol > 0) cid = prow[5 + min(max(col, static_cast<int64_t>(0)), static_cast<int64_t>(ncol - 1))];
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
        if (NEOX) {
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

// One wave per task, capped at the workgroups that fit on the device at once
// (occupancy from the runtime, cached per kernel instance): waves loop over
// their task lists instead of waiting for a second round of workgroups.
template <auto Kernel>
int launch_wave(hipStream_t stream, const GatherArgs& a, int64_t tasks) {
  static int resident = 0;
  if (resident == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, Kernel, kThreads, 0) != hipSuccess || per_cu <= 0) {
      per_cu = 2;
    }
    resident = per_cu * device_cu_count();
  }
  const int64_t wgs = (tasks + kThreads / 64 - 1) / (kThreads / 64);
  const int grid = static_cast<int>(wgs < resident ? wgs : resident);
  if (grid <= 0) return clear_error();
  Kernel<<<grid, kThreads, 0, stream>>>(a);
  return check_launch("ds_rebuild_compact_kv");
}

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
  // Buffer offsets are 32-bit: one slot's raw and working caches and the
  // used cos/sin rows must each stay below 2 GiB.
  const int64_t lim = int64_t{1} << 31;
  vec = vec && D / (2 * V) <= 64 &&
        static_cast<int64_t>(a.max_model_len) * a.heads * D * static_cast<int64_t>(sizeof(T)) < lim &&
        static_cast<int64_t>(a.heads) * a.budget * D * static_cast<int64_t>(sizeof(T)) < lim &&
        static_cast<int64_t>(a.pos_limit) * a.cs_stride * static_cast<int64_t>(sizeof(T)) < lim;
  if (vec) {
    a.lanes_per_row = D / (2 * V);
    const int ppw = 64 / a.lanes_per_row;
    const int64_t tasks = static_cast<int64_t>(a.rows) * ((a.pos_limit + ppw - 1) / ppw);
    if (a.heads >= 4) {
      if (neox) return launch_wave<gather_wave_kernel<DT, true, 4>>(stream, a, tasks);
      return launch_wave<gather_wave_kernel<DT, false, 4>>(stream, a, tasks);
    }
    if (a.heads >= 2) {
      if (neox) return launch_wave<gather_wave_kernel<DT, true, 2>>(stream, a, tasks);
      return launch_wave<gather_wave_kernel<DT, false, 2>>(stream, a, tasks);
    }
    if (neox) return launch_wave<gather_wave_kernel<DT, true, 1>>(stream, a, tasks);
    return launch_wave<gather_wave_kernel<DT, false, 1>>(stream, a, tasks);
  }
  a.lanes_per_row = 1;
  gather_scalar_kernel<DT><<<grid, kThreads, 0, stream>>>(a, neox ? 1 : 0);
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
