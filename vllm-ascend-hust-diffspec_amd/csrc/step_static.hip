// ds_retrieval_step_static: the retrieval step with its scratch memory in a
// static device array instead of caller-provided buffers, for callers that
// cannot allocate (code under HIP graph capture, serving loops that forbid
// allocation).  It allocates nothing and calls no allocating routine.
//
// The array `scratch` lives in this file's code object; each GPU holds its
// own copy, zero-filled when the library's code is loaded, for the life of
// the process.  Host code never uses the array's name as a device address:
// the first call on a device looks its address up with hipGetSymbolAddress
// (with that device current) and keeps it per device.
//
// Fixed regions, so that calls of different shapes and paths never see each
// other's words in the wrong role:
//   [0, 8 MiB)        single-launch workspace: a 64-byte header (epoch,
//                     done counter, status, launch status), tagged plan
//                     copies, task states, tagged partials.  Every word past
//                     the header is tagged with its launch's epoch, which
//                     only grows, so it starts valid from zero and needs no
//                     clearing between calls.
//   [8, 12 MiB)       per-KV-head score partials of the kernel chain, written
//                     before they are read within each call (so SELECT is
//                     refused without SCORE).
//   [12, 24 MiB)      (max, sum) pairs of scoring without a supplied LSE,
//                     written before they are read within each call.
// Calls that overlap on one GPU (two streams, or two threads) race on these
// regions; serialise them.
#include <mutex>

#include "rowdesc.h"

namespace ds355 {

int retrieval_step(hipStream_t stream, const ds_step_desc* d, uint32_t* status_out);
size_t fused_workspace_bytes(int rows, int max_chunks, int num_kv_heads, int token_budget);

namespace {

constexpr size_t kFusedRegion = DS_STATIC_FUSED_BYTES;
constexpr size_t kPartialsRegion = DS_STATIC_PARTIALS_BYTES;
constexpr size_t kPairsRegion = DS_STATIC_PAIRS_BYTES;
constexpr size_t kScratchBytes = kFusedRegion + kPartialsRegion + kPairsRegion;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up once per device).
int device_scratch(char*& out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_error(DS_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  DS_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d is beyond the %d devices the static scratch serves", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      return set_error(DS_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(err));
    }
    g_scratch[dev] = static_cast<char*>(ptr);
  }
  out = g_scratch[dev];
  return DS_OK;
}

}  // namespace

}  // namespace ds355

extern "C" int ds_retrieval_step_static(ds_stream_t stream, const ds_step_desc* d, uint32_t* status) {
  using namespace ds355;
  DS_REQUIRE(d != nullptr, "null step descriptor");
  DS_REQUIRE(d->score_partials == nullptr && d->workspace == nullptr && d->workspace_bytes == 0 &&
                 d->lse_partials == nullptr,
             "the static-scratch step takes no score_partials, workspace or lse_partials (they live in its "
             "static scratch)");
  const bool score = (d->stages & DS_STAGE_SCORE) != 0;
  const bool select = (d->stages & DS_STAGE_SELECT) != 0;
  // Selection reads the per-KV-head partials, which here live in the static
  // array: only a SCORE stage of the same call writes them for this layout.
  DS_REQUIRE(score || !select,
             "the static-scratch step selects only after scoring in the same call (DS_STAGE_SELECT needs "
             "DS_STAGE_SCORE): its score partials live in the static scratch; use ds_retrieval_step with caller "
             "score_partials for a separate selection");
  const int64_t rows = std::max(d->batch_rows, 0);
  const int64_t chunks = std::max(d->max_chunks, 0);
  const int64_t hkv = std::max(d->num_kv_heads, 0);
  const int64_t hq = std::max(d->num_q_heads, 0);

  ds_step_desc s = *d;
  char* base = nullptr;
  if (score || select) {
    const int64_t partial_bytes = rows * chunks * hkv * static_cast<int64_t>(sizeof(float));
    DS_REQUIRE(partial_bytes <= static_cast<int64_t>(kPartialsRegion),
               "static scratch: score partials need %lld bytes (%lld rows x %lld chunks x %lld KV heads x 4), "
               "more than its %zu; use ds_retrieval_step with caller buffers",
               static_cast<long long>(partial_bytes), static_cast<long long>(rows), static_cast<long long>(chunks),
               static_cast<long long>(hkv), kPartialsRegion);
    if (score && d->lse == nullptr) {
      const int64_t pair_bytes = rows * hq * chunks * 2 * static_cast<int64_t>(sizeof(float));
      DS_REQUIRE(pair_bytes <= static_cast<int64_t>(kPairsRegion),
                 "static scratch: scoring without an LSE needs %lld bytes of (max, sum) pairs (%lld rows x %lld "
                 "query heads x %lld chunks x 8), more than its %zu; use ds_retrieval_step with caller buffers",
                 static_cast<long long>(pair_bytes), static_cast<long long>(rows), static_cast<long long>(hq),
                 static_cast<long long>(chunks), kPairsRegion);
    }
    const int rc = device_scratch(base);
    if (rc != DS_OK) return rc;
    s.score_partials = reinterpret_cast<float*>(base + kFusedRegion);
    if (score && d->lse == nullptr) s.lse_partials = reinterpret_cast<float*>(base + kFusedRegion + kPartialsRegion);
    // The single launch when its workspace fits the region; otherwise the
    // chain runs, with the same results.
    const size_t need = fused_workspace_bytes(d->batch_rows, d->max_chunks, d->num_kv_heads, d->token_budget);
    if (d->stages == DS_STAGE_ALL && need > 0 && need <= kFusedRegion) {
      s.workspace = base;
      s.workspace_bytes = kFusedRegion;
    }
  }
  return retrieval_step(reinterpret_cast<hipStream_t>(stream), &s, status);
}
