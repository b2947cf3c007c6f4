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
#include "gather_body.h"
#include "rowdesc.h"

namespace ds355 {
namespace {

using namespace gather;

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
  __shared__ int s_prefix[kMaxRows + 1];
  __shared__ int s_scratch[4];

  const int ppw = 64 / a.lanes_per_row;
  build_row_prefix(a.rows, s_prefix, s_scratch, [&](int r) { return (row_len(a, r) + ppw - 1) / ppw; });
  const int total = s_prefix[a.rows];
  const GatherLane L = gather_lane<DT, NEOX>(a);

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
    gather_task<DT, NEOX, HG>(a, L, p0, slot, len, tail_start, prefix_len, drop,
                              [&](int64_t c) { return prow[5 + c]; });
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

// Where plan rows come from when the gather builds them itself: the
// per-slot selection state and each row's committed length.
struct PlanSource {
  const int32_t* sel_ids;    // [num_slots, sel_stride] ascending chunk ids
  int64_t sel_stride;
  const int32_t* sel_count;  // [num_slots]: -1 none, 0 empty, n ids
  const int32_t* slots;      // [rows]; outside [0, num_slots): padding
  const int32_t* committed;  // [rows] root position + 1
  int64_t* plan;             // [rows, plan_width] output
  int32_t* working_lens;     // [num_slots] output, or nullptr
  int hb, window, cap;       // history budget, rolling tail, chunk ids per plan row (<= 128)
  const int32_t* gen;        // [num_slots] selection generations, or nullptr (no records)
  uint64_t* rec;             // [num_slots, rec_stride] gather records (gather_body.h), or nullptr
  int64_t rec_stride;
  int prefix_only;           // move only tasks wholly in the history prefix
  RowSource src;             // committed lengths from the verifier rows when `committed` is nullptr
};

// Plan and gather of one row in one launch (the compact prefill of
// diffspec/runtime.py:1737-1765 + compact_kv.py:8-133 without a plan kernel
// in between).  Workgroup (r, blk) covers local positions [blk * 4 * ppw,
// (blk + 1) * 4 * ppw) of row r, one task of ppw positions per wave.  Each
// wave derives the row's plan itself (diffspec/runtime.py:1713-1735, the
// arithmetic of write_plan_row): the slot and committed length, then the
// slot's selection count and ids in the same round trip (lane l holds ids l
// and 64 + l), a wave sum for the prefix tokens.  Workgroup (r, 0) stores the
// plan row and working_lens[slot].  Then the wave moves its positions with
// the chunk ids taken from its own registers.
template <int DT, bool NEOX, int HG>
__global__ __launch_bounds__(kThreads) void plan_gather_kernel(GatherArgs a, PlanSource ps) {
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int r = static_cast<int>(blockIdx.y);
  const int ppw = 64 / a.lanes_per_row;
  const int p0 = (static_cast<int>(blockIdx.x) * (kThreads / 64) + wave) * ppw;

  const int slot = scalar_load(ps.slots + r);
  const int committed = ps.committed != nullptr ? scalar_load(ps.committed + r) : committed_of(nullptr, ps.src, r);
  const bool active = a.row_active == nullptr || scalar_load(a.row_active + r) != 0;
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  const bool writer = blockIdx.x == 0 && wave == 0;
  int count = -1;
  uint32_t lo = 0, hi = 0, gen = 0;
  uint64_t have = 0;  // the wave's gather record, requested with the selection
  if (slot_ok) {
    const int32_t* ids = ps.sel_ids + static_cast<int64_t>(slot) * ps.sel_stride;
    count = scalar_load(ps.sel_count + slot);
    if (ps.rec != nullptr) {
      gen = static_cast<uint32_t>(scalar_load(ps.gen + slot));
      have = ps.rec[static_cast<int64_t>(slot) * ps.rec_stride + p0 / ppw];
    }
    lo = lane < ps.cap ? static_cast<uint32_t>(ids[lane]) : 0u;
    hi = lane + 64 < ps.cap ? static_cast<uint32_t>(ids[lane + 64]) : 0u;
  }
  if (!slot_ok) {  // padding row: a zero plan row, nothing gathered
    if (writer) {
      int64_t* prow = ps.plan + static_cast<int64_t>(r) * a.plan_width;
      for (int j = lane; j < a.plan_width; j += 64) prow[j] = 0;
    }
    return;
  }
  const int n = count < 0 ? -1 : min(count, ps.cap);
  const int64_t end = max(0, committed - 1);
  const int64_t hb = ps.hb;
  int64_t len, tail_start, prefix_len = 0, drop = 0;
  if (n < 0) {
    len = min(end, hb);
    tail_start = end - len;
  } else {
    const int64_t tail_len = min(min(end, static_cast<int64_t>(ps.window)), hb);
    tail_start = end - tail_len;
    len = tail_len;
    if (n > 0) {
      const int lastc = n - 1;
      const uint32_t last = lastc < 64 ? __builtin_amdgcn_readlane(lo, lastc) : __builtin_amdgcn_readlane(hi, lastc - 64);
      const int64_t prefix_end = min(tail_start, static_cast<int64_t>(last) * a.chunk);
      auto clipped = [&](uint32_t id, bool in) -> int {
        const int64_t t = prefix_end - static_cast<int64_t>(id) * a.chunk;
        return !in || t <= 0 ? 0 : static_cast<int>(t < a.chunk ? t : a.chunk);
      };
      const int64_t prefix_tokens = wave_sum_int(clipped(lo, lane < n) + clipped(hi, lane + 64 < n));
      prefix_len = min(prefix_tokens, hb - tail_len);
      drop = prefix_tokens - prefix_len;
      len = prefix_len + tail_len;
    }
  }
  if (writer) {
    int64_t* prow = ps.plan + static_cast<int64_t>(r) * a.plan_width;
    const int ncols = max(n, 0);
    // Whole-wave iterations: a lane permute reads only lanes that are active.
    for (int base = 0; base < a.plan_width; base += 64) {
      const int j = base + lane;
      const int c = j - 5;
      const uint32_t lv = __builtin_amdgcn_ds_bpermute((c & 63) << 2, static_cast<int>(lo));
      const uint32_t hv = __builtin_amdgcn_ds_bpermute((c & 63) << 2, static_cast<int>(hi));
      int64_t v;
      if (j == 0) v = slot;
      else if (j == 1) v = len;
      else if (j == 2) v = tail_start;
      else if (j == 3) v = prefix_len;
      else if (j == 4) v = drop;
      else v = c < ncols ? static_cast<int64_t>(c < 64 ? lv : hv) : 0;
      if (j < a.plan_width) prow[j] = v;
    }
    if (lane == 0 && ps.working_lens != nullptr) ps.working_lens[slot] = static_cast<int32_t>(len);
  }
  const int64_t limit = min(len, static_cast<int64_t>(a.pos_limit));
  if (!active) return;
  // The wave's record (its own entry: read before it is rewritten, by this
  // wave only), and whether its task is moved at all.  A task cut by the
  // position limit is not moved whole: no record.  Before the draft's
  // prefill (prefix_only), only a task whose raw rows all precede the rows
  // that prefill rewrites is moved (and recorded).
  const bool early_ok = !ps.prefix_only || sources_final(p0, ppw, tail_start, prefix_len, first_rewritten(ps.src, r));
  const uint64_t want =
      p0 + ppw <= limit && early_ok ? history_record(p0, ppw, len, tail_start, prefix_len, drop, gen) : 0u;
  bool move = p0 < limit && (!ps.prefix_only || want != 0u);
  if (ps.rec != nullptr) {
    have = static_cast<uint64_t>(uniform64(static_cast<int64_t>(have)));
    if (want != 0u && have == want) move = false;
    if (lane == 0 && have != want) ps.rec[static_cast<int64_t>(slot) * ps.rec_stride + p0 / ppw] = want;
  }
  if (!move) return;
  const GatherLane L = gather_lane<DT, NEOX>(a);
  gather_task<DT, NEOX, HG>(a, L, p0, slot, limit, tail_start, prefix_len, drop, [&](int64_t c) {
    const int col = static_cast<int>(c);
    const int l = __builtin_amdgcn_ds_bpermute((col & 63) << 2, static_cast<int>(lo));
    const int h = __builtin_amdgcn_ds_bpermute((col & 63) << 2, static_cast<int>(hi));
    return static_cast<int64_t>(col < 64 ? l : h);
  });
}

// Gather records of the rows' slots set to 0 (nothing known held): one
// workgroup per row, for rebuilds that keep no records.
__global__ __launch_bounds__(kThreads) void clear_records_kernel(const int32_t* slots, int num_slots,
                                                                 const int32_t* row_active, uint64_t* rec,
                                                                 int64_t rec_stride, int64_t entries) {
  const int r = static_cast<int>(blockIdx.x);
  if (row_active != nullptr && row_active[r] == 0) return;
  const int slot = slots[r];
  if (slot < 0 || slot >= num_slots) return;
  for (int64_t i = threadIdx.x; i < entries; i += kThreads) rec[slot * rec_stride + i] = 0u;
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

// Whether the vector path covers these shapes and pointers; sets
// lanes_per_row (1 for the scalar path).
template <int DT>
bool vector_path(GatherArgs& a, bool neox) {
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
  a.lanes_per_row = vec ? D / (2 * V) : 1;
  return vec;
}

template <int DT>
int launch_gather(hipStream_t stream, const GatherArgs& a, bool neox, bool vec, int grid) {
  if (vec) {
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
  gather_scalar_kernel<DT><<<grid, kThreads, 0, stream>>>(a, neox ? 1 : 0);
  return check_launch("ds_rebuild_compact_kv");
}

template <int DT>
int launch_plan_gather_dt(hipStream_t stream, const GatherArgs& a, const PlanSource& ps, bool neox) {
  const int ppw = 64 / a.lanes_per_row;
  const int per_wg = (kThreads / 64) * ppw;
  const dim3 grid(static_cast<unsigned>(std::max(1, (a.pos_limit + per_wg - 1) / per_wg)),
                  static_cast<unsigned>(a.rows));
  if (a.heads >= 4) {
    if (neox) plan_gather_kernel<DT, true, 4><<<grid, kThreads, 0, stream>>>(a, ps);
    else plan_gather_kernel<DT, false, 4><<<grid, kThreads, 0, stream>>>(a, ps);
  } else if (a.heads >= 2) {
    if (neox) plan_gather_kernel<DT, true, 2><<<grid, kThreads, 0, stream>>>(a, ps);
    else plan_gather_kernel<DT, false, 2><<<grid, kThreads, 0, stream>>>(a, ps);
  } else {
    if (neox) plan_gather_kernel<DT, true, 1><<<grid, kThreads, 0, stream>>>(a, ps);
    else plan_gather_kernel<DT, false, 1><<<grid, kThreads, 0, stream>>>(a, ps);
  }
  return check_launch("plan + gather");
}

}  // namespace

int make_gather_args(GatherArgs& a, bool& vec, int& scalar_grid, int dtype, const void* raw_key,
                     const void* raw_value, void* working_key, void* working_value, const int64_t* plan, int rows,
                     int plan_width, const void* cos_sin, int64_t cs_stride, int cs_rows, int num_slots,
                     int max_model_len, int heads, int head_dim, int token_budget, int chunk_size, int rotary_dim,
                     int is_neox_style, int max_width, const int32_t* row_active, bool padded_rows) {
  a = GatherArgs{};
  vec = false;
  scalar_grid = 0;
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
  scalar_grid = static_cast<int>(max_tiles < cap ? max_tiles : cap);
  const bool neox = is_neox_style != 0;
  switch (dtype) {
    case DS_BF16: vec = vector_path<DS_BF16>(a, neox); break;
    case DS_FP16: vec = vector_path<DS_FP16>(a, neox); break;
    default: vec = vector_path<DS_FP32>(a, neox); break;
  }
  return clear_error();
}

int rebuild_compact_kv_impl(hipStream_t stream, int dtype, const void* raw_key, const void* raw_value,
                            void* working_key, void* working_value, const int64_t* plan, int rows,
                            int plan_width, const void* cos_sin, int64_t cs_stride, int cs_rows, int num_slots,
                            int max_model_len, int heads, int head_dim, int token_budget, int chunk_size,
                            int rotary_dim, int is_neox_style, int max_width, const int32_t* row_active,
                            bool padded_rows) {
  GatherArgs a;
  bool vec = false;
  int grid = 0;
  const int rc = make_gather_args(a, vec, grid, dtype, raw_key, raw_value, working_key, working_value, plan, rows,
                                  plan_width, cos_sin, cs_stride, cs_rows, num_slots, max_model_len, heads, head_dim,
                                  token_budget, chunk_size, rotary_dim, is_neox_style, max_width, row_active,
                                  padded_rows);
  if (rc != DS_OK || grid <= 0) return rc;
  const bool neox = is_neox_style != 0;
  switch (dtype) {
    case DS_BF16: return launch_gather<DS_BF16>(stream, a, neox, vec, grid);
    case DS_FP16: return launch_gather<DS_FP16>(stream, a, neox, vec, grid);
    default: return launch_gather<DS_FP32>(stream, a, neox, vec, grid);
  }
}

// Plans from the slot selections and the gather, as one launch.  Sets
// `launched` when it ran; shapes the vector path does not cover (or more
// than 128 chunk ids per plan row) launch nothing, and the caller runs the
// plan kernel and the gather instead.
int launch_plan_gather(hipStream_t stream, int dtype, const void* raw_key, const void* raw_value,
                       void* working_key, void* working_value, int rows, int plan_width, const void* cos_sin,
                       int64_t cs_stride, int cs_rows, int num_slots, int max_model_len, int heads, int head_dim,
                       int token_budget, int chunk_size, int rotary_dim, int is_neox_style, int history_budget,
                       const int32_t* row_active, const int32_t* sel_ids, int64_t sel_stride,
                       const int32_t* sel_count, const int32_t* slots, const int32_t* committed_lens, int64_t* plan,
                       int32_t* working_lens, int recent_window, const int32_t* gen, uint64_t* rec,
                       int64_t rec_stride, bool prefix_only, const RowSource& src, bool& launched) {
  launched = false;
  GatherArgs a;
  bool vec = false;
  int grid = 0;
  int rc = make_gather_args(a, vec, grid, dtype, raw_key, raw_value, working_key, working_value, plan, rows,
                            plan_width, cos_sin, cs_stride, cs_rows, num_slots, max_model_len, heads, head_dim,
                            token_budget, chunk_size, rotary_dim, is_neox_style, history_budget, row_active, true);
  if (rc != DS_OK) return rc;
  const int64_t cap = std::min<int64_t>(plan_width - 5, sel_stride);
  if (rows == 0 || !vec || cap > 128 || grid <= 0) return clear_error();
  DS_REQUIRE(sel_ids && sel_count && slots && plan && (committed_lens || src.counts), "null plan pointer");
  DS_REQUIRE(recent_window > 0, "recent_window must be positive");
  DS_REQUIRE(history_budget >= chunk_size && history_budget % chunk_size == 0,
             "history_budget must be a positive chunk-size multiple");
  PlanSource ps{};
  ps.sel_ids = sel_ids;
  ps.sel_stride = sel_stride;
  ps.sel_count = sel_count;
  ps.slots = slots;
  ps.committed = committed_lens;
  ps.plan = plan;
  ps.working_lens = working_lens;
  ps.hb = history_budget;
  ps.window = recent_window;
  ps.cap = static_cast<int>(cap);
  if (rec != nullptr) {
    DS_REQUIRE(gen != nullptr, "gather records need the selection generations");
    DS_REQUIRE(rec_stride >= token_budget, "gather record row stride is smaller than token_budget");
  }
  ps.gen = gen;
  ps.rec = rec;
  ps.rec_stride = rec_stride;
  ps.prefix_only = prefix_only ? 1 : 0;
  ps.src = src;
  const bool neox = is_neox_style != 0;
  switch (dtype) {
    case DS_BF16: rc = launch_plan_gather_dt<DS_BF16>(stream, a, ps, neox); break;
    case DS_FP16: rc = launch_plan_gather_dt<DS_FP16>(stream, a, ps, neox); break;
    default: rc = launch_plan_gather_dt<DS_FP32>(stream, a, ps, neox); break;
  }
  launched = rc == DS_OK;
  return rc;
}

int clear_gather_records(hipStream_t stream, const int32_t* slots, int rows, int num_slots,
                         const int32_t* row_active, uint64_t* rec, int64_t rec_stride, int64_t entries) {
  if (rows <= 0) return clear_error();
  DS_SUPPORTED(rows <= 65535, "at most 65535 rows per launch");
  clear_records_kernel<<<rows, kThreads, 0, stream>>>(slots, num_slots, row_active, rec, rec_stride, entries);
  return check_launch("clear gather records");
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
