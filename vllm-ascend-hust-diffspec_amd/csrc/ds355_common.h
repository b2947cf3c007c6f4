// Shared device helpers and host-side error plumbing for libds355.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <climits>

#include "../../include/ds355.h"

namespace ds355 {

// ---------------------------------------------------------------------------
// Host: thread-local error message and argument checks.
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int clear_error();
int check_launch(const char* what);

#define DS_REQUIRE(cond, ...)                              \
  do {                                                     \
    if (!(cond)) return ::ds355::set_error(DS_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define DS_SUPPORTED(cond, ...)                            \
  do {                                                     \
    if (!(cond)) return ::ds355::set_error(DS_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)

// Compute units of the current device (cached per device).
int device_cu_count();

// Upper bound on rows handled by one launch (LDS prefix arrays).
constexpr int kMaxRows = 1024;

// ---------------------------------------------------------------------------
// Device: element conversions.  bf16 / fp16 are carried as raw 16-bit words.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even; NaN -> 0x7fc0 (the CPU oracle's rule).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> fp16, IEEE round to nearest even.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Element traits: storage word, widening to fp32 and rounding back.
template <int DT> struct Elem;
template <> struct Elem<DS_BF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(T v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ T store(float f) { return f32_to_bf16(f); }
};
template <> struct Elem<DS_FP16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(T v) { return f16_to_f32(v); }
  static __device__ __forceinline__ T store(float f) { return f32_to_f16(f); }
};
template <> struct Elem<DS_FP32> {
  using T = float;
  static __device__ __forceinline__ float load(T v) { return v; }
  static __device__ __forceinline__ T store(float f) { return f; }
};

// ---------------------------------------------------------------------------
// Device: wave64 reductions and block-wide exclusive scan over 256 threads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over the 64 lanes with DPP lane permutes only (no LDS instruction, so
// it never waits on outstanding scalar or LDS loads).  The total lands in
// lane 63.  Steps: quad xor 1, quad xor 2, half-row mirror, row mirror (each
// 16-lane row now holds its row sum), then row broadcasts 15 and 31 fold the
// four rows into row 3.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true));
}
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Load through the constant address space: a wave-uniform address becomes a
// scalar (SMEM) load, counted by lgkmcnt instead of the in-order vmcnt, so
// waiting for it never drains vector loads in flight.  Only for memory the
// kernel does not write (a launch starts with the scalar cache invalidated,
// so data written by an earlier kernel on the stream is seen).
__device__ __forceinline__ int32_t scalar_load(const int32_t* p) {
  typedef const __attribute__((address_space(4))) int32_t* const_ptr;
  return *(const_ptr)(p);
}
__device__ __forceinline__ int64_t scalar_load(const int64_t* p) {
  typedef const __attribute__((address_space(4))) int64_t* const_ptr;
  return *(const_ptr)(p);
}

// Device-scope (coherent) loads and stores: relaxed atomics at agent scope,
// which read and write past the per-XCD L2 caches.  Used for values that
// workgroups of one launch hand to each other.
template <typename T>
__device__ __forceinline__ T coherent_load(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void coherent_store(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wave-uniform 64-bit value made scalar (both halves through readfirstlane).
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Workgroup barrier for LDS hand-offs only.  Unlike __syncthreads it does
// not wait for the wave's outstanding global loads, stores and atomics, which
// the other waves of the workgroup do not read.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Inclusive scan within the wave (lane order), with DPP lane moves only:
// row shifts by 1, 2, 4, 8 scan each 16-lane row (lanes without a source
// add 0), then row broadcasts of lanes 15 and 31 carry the row totals into
// rows 1, 3 and 2, 3.  The whole wave must be active.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_add_int(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v = dpp_add_int<0x111, 0xf>(v);  // row_shr:1
  v = dpp_add_int<0x112, 0xf>(v);  // row_shr:2
  v = dpp_add_int<0x114, 0xf>(v);  // row_shr:4
  v = dpp_add_int<0x118, 0xf>(v);  // row_shr:8
  v = dpp_add_int<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add_int<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}
// Largest / smallest unsigned value over the wave, in every lane: the same
// DPP steps as the scan with max / min in place of add (a lane without a
// source combines with the identity).
template <int CTRL, int ROW_MASK, bool MAX>
__device__ __forceinline__ uint32_t dpp_pick(uint32_t v) {
  const uint32_t other = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(MAX ? 0u : ~0u), static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
  return MAX ? max(v, other) : min(v, other);
}
template <bool MAX>
__device__ __forceinline__ uint32_t wave_pick(uint32_t v) {
  v = dpp_pick<0x111, 0xf, MAX>(v);
  v = dpp_pick<0x112, 0xf, MAX>(v);
  v = dpp_pick<0x114, 0xf, MAX>(v);
  v = dpp_pick<0x118, 0xf, MAX>(v);
  v = dpp_pick<0x142, 0xa, MAX>(v);
  v = dpp_pick<0x143, 0xc, MAX>(v);
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Sum over the wave, in every lane (the scan's lane 63).
__device__ __forceinline__ int wave_total(int v) {
  return __builtin_amdgcn_readlane(wave_inclusive_scan(v), 63);
}

// Exclusive scan over a 256-thread block; `total` receives the block sum.
// Uses scratch[4]; contains two barriers.
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int inc = wave_inclusive_scan(v);
  if (lane == 63) scratch[wave] = inc;
  __syncthreads();
  int base = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    int s = scratch[w];
    if (w < wave) base += s;
    total += s;
  }
  __syncthreads();
  return base + inc - v;
}

// Row prefix table in LDS: prefix[i] = sum_{j<i} count(j), for i <= rows.
// Built by a 256-thread block in chunks of 256 rows.  Ends with a barrier.
template <typename CountFn>
__device__ __forceinline__ void build_row_prefix(int rows, int* prefix, int* scratch, CountFn count) {
  int carry = 0;
  for (int base = 0; base < rows; base += 256) {
    const int r = base + static_cast<int>(threadIdx.x);
    const int c = r < rows ? count(r) : 0;
    int total;
    const int ex = block_exclusive_scan(c, scratch, total);
    if (r < rows) prefix[r] = carry + ex;
    carry += total;
  }
  if (threadIdx.x == 0) prefix[rows] = carry;
  __syncthreads();
}

// Largest i in [0, rows) with prefix[i] <= unit (prefix is non-decreasing,
// prefix[0] == 0 and unit < prefix[rows]).
__device__ __forceinline__ int find_row(const int* prefix, int rows, int unit) {
  int lo = 0, hi = rows - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= unit) lo = mid; else hi = mid - 1;
  }
  return lo;
}

}  // namespace ds355
