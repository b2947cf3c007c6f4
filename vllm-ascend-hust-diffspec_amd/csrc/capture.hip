// Raw pre-RoPE K/V capture of draft tokens and the graph-safe RoPE input, in
// one launch.
//
// Counterpart of DiffSpecDraftCache._write_raw (diffspec/runtime.py:1602-1618),
// the local-position part of capture_raw_kv (:1797-1877) and
// graph_safe_rope_positions (:1767-1794).  The reference builds index tensors
// on the host and runs torch index_put / copy / zero ops; here:
//   - token t < tokens: raw[token_slots[t], positions[t], h, :] = key[t, h, :]
//     (and value), for every KV head h;
//   - RoPE input rope[t] for t < count: positions[t] (absolute mode), or
//     local[t] (explicit local positions), or, for t < tokens,
//     working_lens[token_slots[t]] (the draft rows' local positions; the
//     rows past `tokens` are graph padding and get 0);
//   - rope[t] = 0 for count <= t < prev_count (the stale tail of the previous
//     call, so a larger graph bucket never reads old positions).
// A wave moves one token row (both caches), as 16-byte vectors when rows,
// strides and pointers allow, else element by element; threads also cover
// the RoPE entries.  Tokens whose slot or position is out of range are not written
// and set bit 0 of *status (when given).
#include "ds355_common.h"

namespace ds355 {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreadsC = 256;
constexpr int kWavesC = kThreadsC / 64;

struct CaptureArgs {
  const uint8_t* key;
  const uint8_t* value;
  int64_t k_row, k_head, v_row, v_head;  // bytes
  const void* positions;
  int index64;
  const int32_t* token_slots;
  int tokens;
  uint8_t* raw_key;
  uint8_t* raw_value;
  int num_slots, max_model_len, heads;
  int row_bytes;  // head_dim * element size
  int elem;       // element size
  int vec;        // rows, strides and pointers are whole 16-byte vectors
  const int32_t* working_lens;
  const void* local;
  void* rope;
  int count, prev_count;
  int32_t* status;
};

__device__ __forceinline__ int64_t read_index(const void* p, int index64, int t) {
  return index64 ? static_cast<const int64_t*>(p)[t] : static_cast<int64_t>(static_cast<const int32_t*>(p)[t]);
}

__device__ __forceinline__ void write_index(void* p, int index64, int t, int64_t v) {
  if (index64) static_cast<int64_t*>(p)[t] = v;
  else static_cast<int32_t*>(p)[t] = static_cast<int32_t>(v);
}

__global__ __launch_bounds__(kThreadsC) void capture_kernel(CaptureArgs a) {
  // RoPE input (and the stale tail).
  const int i = blockIdx.x * kThreadsC + threadIdx.x;
  if (i < max(a.count, a.prev_count)) {
    int64_t v = 0;
    if (i < a.count) {
      if (a.working_lens) {
        if (i < a.tokens) {
          const int slot = a.token_slots[i];
          v = (slot >= 0 && slot < a.num_slots) ? a.working_lens[slot] : 0;
        }
      } else {
        v = read_index(a.local ? a.local : a.positions, a.index64, i);
      }
    }
    write_index(a.rope, a.index64, i, v);
  }

  // Raw K/V rows: one wave per token, 16-byte vectors over the heads.
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kWavesC + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  const int slot = a.token_slots[t];
  const int64_t pos = read_index(a.positions, a.index64, t);
  if (slot < 0 || slot >= a.num_slots || pos < 0 || pos >= a.max_model_len) {
    if (lane == 0 && a.status) __hip_atomic_fetch_or(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int64_t dst_row = ((static_cast<int64_t>(slot) * a.max_model_len + pos) * a.heads) * a.row_bytes;
  if (a.vec) {
    const int vecs = a.row_bytes / 16;  // per head
    for (int e = lane; e < a.heads * vecs; e += 64) {
      const int h = e / vecs, c = e % vecs;
      const u32x4 kv = *reinterpret_cast<const u32x4*>(a.key + t * a.k_row + h * a.k_head + 16 * c);
      const u32x4 vv = *reinterpret_cast<const u32x4*>(a.value + t * a.v_row + h * a.v_head + 16 * c);
      *reinterpret_cast<u32x4*>(a.raw_key + dst_row + static_cast<int64_t>(h) * a.row_bytes + 16 * c) = kv;
      *reinterpret_cast<u32x4*>(a.raw_value + dst_row + static_cast<int64_t>(h) * a.row_bytes + 16 * c) = vv;
    }
  } else {  // rows that are not whole 16-byte vectors: element by element
    const int elems = a.row_bytes / a.elem;  // per head
    for (int e = lane; e < a.heads * elems; e += 64) {
      const int h = e / elems, c = e % elems;
      const int64_t src_k = t * a.k_row + h * a.k_head + c * a.elem;
      const int64_t src_v = t * a.v_row + h * a.v_head + c * a.elem;
      const int64_t dst = dst_row + static_cast<int64_t>(h) * a.row_bytes + c * a.elem;
      if (a.elem == 4) {
        *reinterpret_cast<uint32_t*>(a.raw_key + dst) = *reinterpret_cast<const uint32_t*>(a.key + src_k);
        *reinterpret_cast<uint32_t*>(a.raw_value + dst) = *reinterpret_cast<const uint32_t*>(a.value + src_v);
      } else {
        *reinterpret_cast<uint16_t*>(a.raw_key + dst) = *reinterpret_cast<const uint16_t*>(a.key + src_k);
        *reinterpret_cast<uint16_t*>(a.raw_value + dst) = *reinterpret_cast<const uint16_t*>(a.value + src_v);
      }
    }
  }
}

int elem_bytes(int dtype) { return dtype == DS_FP32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int capture_impl(hipStream_t stream, int dtype, const void* key, int64_t k_row, int64_t k_head, const void* value,
                 int64_t v_row, int64_t v_head, const void* positions, int index64, const int32_t* token_slots,
                 int tokens, void* raw_key, void* raw_value, int num_slots, int max_model_len, int heads,
                 int head_dim, const int32_t* working_lens, const void* local_positions, void* rope, int count,
                 int prev_count, int32_t* status) {
  DS_REQUIRE(dtype == DS_BF16 || dtype == DS_FP16 || dtype == DS_FP32, "KV caches must use BF16, FP16 or FP32");
  DS_REQUIRE(tokens >= 0 && count >= 0 && prev_count >= 0, "token counts must be non-negative");
  DS_REQUIRE(tokens <= count || count == 0, "captured tokens exceed the position count");
  DS_REQUIRE(num_slots > 0 && max_model_len > 0 && heads > 0 && head_dim > 0,
             "raw sequence, head and head dimensions must be positive");
  DS_REQUIRE(!(working_lens && local_positions), "give working lengths or local positions, not both");
  const int eb = elem_bytes(dtype);
  DS_REQUIRE(tokens == 0 || (key && value && raw_key && raw_value && token_slots && positions),
             "null tensor pointer");
  DS_REQUIRE(max(count, prev_count) == 0 || rope, "null RoPE position buffer");
  DS_REQUIRE(count == 0 || working_lens || local_positions || positions, "null position pointer");
  const bool vec = (head_dim * eb) % 16 == 0 && aligned16(key) && aligned16(value) && aligned16(raw_key) &&
                   aligned16(raw_value) && (k_row * eb) % 16 == 0 && (k_head * eb) % 16 == 0 &&
                   (v_row * eb) % 16 == 0 && (v_head * eb) % 16 == 0;
  const int span = max(count, prev_count);
  const int blocks = max((tokens + kWavesC - 1) / kWavesC, (span + kThreadsC - 1) / kThreadsC);
  if (blocks == 0) return clear_error();
  CaptureArgs a{};
  a.key = static_cast<const uint8_t*>(key);
  a.value = static_cast<const uint8_t*>(value);
  a.k_row = k_row * eb;
  a.k_head = k_head * eb;
  a.v_row = v_row * eb;
  a.v_head = v_head * eb;
  a.positions = positions;
  a.index64 = index64 ? 1 : 0;
  a.token_slots = token_slots;
  a.tokens = tokens;
  a.raw_key = static_cast<uint8_t*>(raw_key);
  a.raw_value = static_cast<uint8_t*>(raw_value);
  a.num_slots = num_slots;
  a.max_model_len = max_model_len;
  a.heads = heads;
  a.row_bytes = head_dim * eb;
  a.elem = eb;
  a.vec = vec ? 1 : 0;
  a.working_lens = working_lens;
  a.local = local_positions;
  a.rope = rope;
  a.count = count;
  a.prev_count = prev_count;
  a.status = status;
  capture_kernel<<<blocks, kThreadsC, 0, stream>>>(a);
  return check_launch("ds_capture_raw_kv");
}

}  // namespace
}  // namespace ds355

extern "C" int ds_capture_raw_kv(ds_stream_t stream, int dtype, const void* key, int64_t k_row_stride,
                                 int64_t k_head_stride, const void* value, int64_t v_row_stride, int64_t v_head_stride,
                                 const void* positions, int positions_int64, const int32_t* token_slots, int tokens,
                                 void* raw_key, void* raw_value, int num_slots, int max_model_len, int heads,
                                 int head_dim, const int32_t* working_lens, const void* local_positions,
                                 void* rope_positions, int count, int prev_count, int32_t* status) {
  return ds355::capture_impl(reinterpret_cast<hipStream_t>(stream), dtype, key, k_row_stride, k_head_stride, value,
                             v_row_stride, v_head_stride, positions, positions_int64, token_slots, tokens, raw_key,
                             raw_value, num_slots, max_model_len, heads, head_dim, working_lens, local_positions,
                             rope_positions, count, prev_count, status);
}
