// One retrieval step (score -> select -> plan -> gather) as a single
// persistent launch.
//
// The three-kernel chain pays each kernel's ramp and drain and leaves the
// device idle while one workgroup per row selects.  Here the stages hand
// work over through memory inside one launch:
//   - workgroups [0, G - S) score: they stream the scored keys exactly as
//     chunk_score_kernel does (units numbered row-major and dealt
//     round-robin, so rows finish roughly in order), then each wave takes its
//     gather tasks, (row, ppw local positions) numbered row-major and dealt
//     round-robin, each once its row's plan is published;
//   - the last S workgroups select: selector s takes rows s, s + S, ... in
//     order and publishes each row's plan (without a supplied LSE, below
//     them the group workgroups; see below).
//
// Hand-over is by value through device-scope (coherent) accesses, with no
// cache write-back on either side:
//   - a score partial is stored as (tag << 32) | fp32 bits.  `tag` is unique
//     to the launch, so stale values of earlier launches never match.  A
//     selector reads the row's partials, 16 per thread at a time, until all
//     carry the tag;
//   - without a supplied LSE (the LSEFREE kernel) the scoring waves store a
//     mass word per (chunk, query head) instead, tagged the same way, in the
//     caller's lse_partials.  Group workgroups, one per (row slot, KV
//     group), sit below the row selectors: each polls its group's sentinel
//     word (newest chunk, last head of the group), merges the group's words
//     into its heads' LSEs and stores each chunk's share of the group as the
//     tagged partial above (lse_finalize_kernel's steps: the same bits); the
//     row's selector then selects as with a supplied LSE.  The words carry
//     the tags of this workspace's launches, so one lse_partials buffer
//     serves one workspace;
//   - a selector stores the plan row twice: as the output (plain stores) and
//     as a tagged copy, column j as (tag << 32) | value (plan values are
//     below 2^31).  Gathering waves poll the tagged copy itself with one
//     wave-wide load (lane l, columns l and 64 + l): it is valid once every
//     column carries the tag, so no flag, and no wait for the stores to
//     complete, stands between a plan and its gathers;
//   - a wave that gave up waiting for a plan stores state[row][task] =
//     tag | kSkipped for each task it left, and sets the launch's skip word.
// Polling is the costly part of this design: every poll is a device-scope
// request to one memory channel, and thousands of waves polling one line
// slow every stream that shares the channel.  So each row's tagged plan has
// lines of its own and polls sleep between tries.  The row selectors (at
// most kSelectors, each on one row at a time) poll their rows' partials
// whole: at most kSelectors rows of partials per round trip (8 KB for a
// 16k-token row with 4 KV heads), and no round trip for a sentinel word
// between the row's last partial and its selection.
//
// Forward progress does not depend on all workgroups being resident at once
// (the launch is an ordinary one).  Workgroups are dispatched in index order
// on each XCD, and a workgroup waits without a deadline only on lower-indexed
// ones: selectors on scorers (partials) and on nobody else.  Scorers wait
// for plans, held by higher-indexed selectors, only up to kOwnerSpins polls;
// a task they give up on is marked skipped and redone by the last workgroup
// to finish, when every plan is published.  A gather task writes fixed bytes
// that depend only on the published plan, so doing one twice is harmless.  The waits without a
// deadline still end after kSpinLimit polls (then a status bit is set and
// the results are not valid), so every wave of the launch finishes.
//
// The tag is the workspace epoch + 1.  The last workgroup to finish (a
// device-scope counter) stores the tag as the new epoch, so graph replays of
// the launch get fresh tags.  Tags stay below 2^31 (bit 31 marks skipped
// tasks).
//
// Status: an expired wait ORs a bit into the launch's own status word
// (header[3]), which every bounded wait of that launch reads to stop early.
// The last workgroup moves those bits into the owner's status word
// (header[2], cleared only by the owner) and zeroes header[3], so one
// launch's expiry never shortens the waits of the next.
//
// Workspace (zero-filled once by its owner; one launch at a time):
//   uint32 header[16]               epoch, done counter, status, launch status, skips
//   uint64 plans[rows][kPlanCols]   tagged plan copies
//   uint32 state[rows][task_cap]    gather tasks skipped by their scoring wave
//   uint64 partials[rows, max_chunks, Hkv]
// (and, without a supplied LSE, the tagged mass words in lse_partials).
#include "gather_body.h"
#include "score_body.h"
#include "select_body.h"

namespace ds355 {

int make_score_args(score::ScoreArgs& a, int64_t& upper_units, int& page_mode, int dtype, const void* query,
                    int64_t q_stride, const void* key_cache, int64_t k_block_stride, int64_t k_token_stride,
                    int64_t k_head_stride, const float* lse, int64_t lse_row_stride, int64_t lse_head_stride,
                    const int32_t* block_table, int64_t bt_stride, const RowSource& src, int batch, int num_q_heads,
                    int num_kv_heads, int head_dim, int block_size, int chunk_size, int max_chunks, float scale,
                    int head_reduce, float* partial, float* out, int64_t out_stride, int write_tail,
                    size_t partial_bytes, uint64_t* mw);
int make_select_args(select::SelectArgs& a, float* scores, int64_t score_stride, const float* partials,
                     int max_chunks, int hkv, int hq, const RowSource& src, int batch, int chunk, int budget,
                     int do_select, int do_plan, int32_t* ids, int64_t ids_stride, int32_t* counts,
                     const int32_t* slots, int num_slots, const int32_t* committed_lens, int64_t* plan,
                     int plan_width, int32_t* working_lens, int recent_window);
int make_gather_args(gather::GatherArgs& a, bool& vec, int& scalar_grid, int dtype, const void* raw_key,
                     const void* raw_value, void* working_key, void* working_value, const int64_t* plan, int rows,
                     int plan_width, const void* cos_sin, int64_t cs_stride, int cs_rows, int num_slots,
                     int max_model_len, int heads, int head_dim, int token_budget, int chunk_size, int rotary_dim,
                     int is_neox_style, int max_width, const int32_t* row_active, bool padded_rows);

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// Row selectors (fewer when the batch has fewer rows).  8 against 16, events
// around each launch, two rounds: 16 rows of 4k-40k tokens 82.5-82.7 against
// 82.8-83.4 us (other seeds 0.3-1.4 us faster), 16 x 40k 156.2-156.4
// against 157.1-157.6 us, 64 rows equal or faster.  A selector's rows
// complete tens of microseconds apart, and the freed slots score.  4
// selectors: 0.5-0.9 us slower on the first draw, up to 1 us faster on
// others; 2: 25-45% slower on ragged rows (selections queue).
constexpr int kSelectors = 8;
// Without a supplied LSE: workgroups doing the KV groups' shares, below the
// row selectors.  Measured on 16 rows of 4k-40k tokens (one step): 32 group
// workgroups 96.6-98.3 us; 16 of them 101.9 us; 32 with the last group's
// workgroup also selecting (no row selectors) 107.7 us; one per row and
// group (64), the last selecting, 103.5 us.  Workgroups that do not score
// lengthen the scoring stream's tail.
constexpr int kGroupSelectors = 32;
constexpr int kFusedKeys = 8192;   // candidate keys a selector keeps in LDS
constexpr int kFusedRows = 256;    // batch rows per fused launch
static_assert(kFusedRows <= kThreads, "the prologue loads one row per thread");
// Fewer rows than this run the chain: the single launch gains by hiding
// rows' selections and gathers behind other rows' scoring, and with a few
// long rows the last selection dominates (measured: 4 rows of 128k tokens
// 157 µs single launch against 130 µs chain; one 8k row 27 against 21).
constexpr int kMinFusedRows = 8;
constexpr int kPollLoads = 16;     // partials per thread polled together (kPollLoads / Hkv chunks)
constexpr int kMaxHkv = 8;         // KV heads the fused kernel takes
constexpr int kGatherHeads = 4;    // heads in flight per gather task
constexpr int kMinTaskPositions = 8;  // ppw >= 8 for the fused shapes: task_cap = ceil(token_budget / 8)
constexpr uint32_t kSpinLimit = 1u << 21;   // polls before a wait without deadline gives up (~2 s)
constexpr uint32_t kOwnerSpins = 1u << 12;  // polls before a scorer leaves a task to the selector (~4 ms)
constexpr uint32_t kSkipped = 0x80000000u;
constexpr int kSleep = 8;          // s_sleep units (64 cycles each) between polls

enum { kEpoch = 0, kDone = 1, kStatus = 2, kLaunchStatus = 3, kSkips = 4, kHeaderWords = 16 };
enum { kStatusPartials = 1u, kStatusTasks = 2u };
constexpr int kLine = 256;
constexpr int kPlanCols = 128;     // tagged plan columns per row (plan_width <= 128)
constexpr int kStatusEvery = 256;  // polls between looks at the shared status word

struct FusedArgs {
  score::ScoreArgs s;
  select::SelectArgs p;
  gather::GatherArgs g;
  uint32_t* header;
  uint64_t* plans;  // [rows, kPlanCols] tagged plan copies
  uint32_t* state;  // [rows, task_cap]
  int task_cap;
  int selectors;        // workgroups that do not score: group workgroups, then row selectors
  int group_selectors;  // of them, LSEFREE: one per (row slot, KV group), below the row selectors
  uint32_t owner_spins;  // polls a scorer waits for a plan (0: every task goes to the selectors)
  int expire;            // test flag: every selector raises kStatusPartials as if a wait had expired
  uint32_t* status_out;  // optional caller word that also receives the launch's status bits
  int32_t* gen;          // [num_slots] selection generations, or nullptr (no gather records)
  uint64_t* rec;         // [num_slots, rec_stride] gather records (gather_body.h), or nullptr
  int64_t rec_stride;
  int prefix_only;       // gather only the tasks wholly in each row's history prefix
  // Without a supplied LSE (the LSEFREE kernel): a selector per (row, KV
  // group) merges the group's mass words (s.mw, tagged) into its heads'
  // LSEs, written to lse_out, and stores the group's tagged partials.
  float* lse_out;
  int64_t lse_out_stride;
  int lse_wide;  // two heads per thread and 16-byte reads (words 16-byte aligned)
};
// With gather records, the tagged plan copy carries the slot's selection
// generation in its last column (plan_width < kPlanCols then).
constexpr int kGenCol = 127;

// The read-modify-write completes before the thread goes on (acquire: the
// wave waits for its return), so the bit is in memory before the workgroup
// counts itself done.  No release: that would write back the XCD's L2.
__device__ __forceinline__ void raise_status(uint32_t* header, uint32_t bit) {
  __hip_atomic_fetch_or(header + kLaunchStatus, bit, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
// A wait without deadline gives up after kSpinLimit polls, or early once
// another wait of this launch has.
__device__ __forceinline__ bool give_up(uint32_t spin, const uint32_t* header) {
  return spin >= kSpinLimit ||
         (spin % kStatusEvery == kStatusEvery - 1 &&
          __builtin_amdgcn_readfirstlane(coherent_load(header + kLaunchStatus)) != 0u);
}

// Waits (one load per wave and poll) until *p carries the tag.
__device__ __forceinline__ void wait_sentinel(const uint64_t* p, uint32_t tag, uint32_t* header) {
  for (uint32_t spin = 0;; ++spin) {
    const uint64_t v = static_cast<uint64_t>(uniform64(static_cast<int64_t>(coherent_load(p))));
    if (static_cast<uint32_t>(v >> 32) == tag) return;
    if (give_up(spin, header)) {
      raise_status(header, kStatusPartials);
      return;
    }
    __builtin_amdgcn_s_sleep(kSleep);
  }
}

// Head sums of chunks base + u * kThreads + tid (u < kPollLoads / hkv,
// below C), in head order, once all of their partials carry `tag`.  The
// kPollLoads loads of a poll are issued together.
__device__ __forceinline__ void poll_chunk_sums(const uint64_t* part, int base, int C, int hkv, uint32_t tag,
                                                uint32_t* header, float (&sum)[kPollLoads]) {
  const int per_chunk = hkv;  // loads per chunk; kPollLoads / hkv chunks per thread
  uint64_t v[kPollLoads] = {};
  for (uint32_t spin = 0;; ++spin) {
    bool ready = true;
#pragma unroll
    for (int e = 0; e < kPollLoads; ++e) {
      const int u = e / per_chunk, g = e - u * per_chunk;
      const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
      if (i < C) v[e] = coherent_load(part + static_cast<int64_t>(i) * hkv + g);
    }
#pragma unroll
    for (int e = 0; e < kPollLoads; ++e) {
      const int u = e / per_chunk;
      const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
      if (i < C && static_cast<uint32_t>(v[e] >> 32) != tag) ready = false;
    }
    if (ready) break;
    if (spin >= kSpinLimit ||
        (spin % kStatusEvery == kStatusEvery - 1 && coherent_load(header + kLaunchStatus) != 0u)) {
      raise_status(header, kStatusPartials);
      break;
    }
    __builtin_amdgcn_s_sleep(kSleep);
  }
  // sum[u] = chunk u's head sum, heads added in order.
#pragma unroll
  for (int u = 0; u < kPollLoads; ++u) sum[u] = 0.f;
#pragma unroll
  for (int e = 0; e < kPollLoads; ++e) {
    const int u = e / per_chunk;
    sum[u] += __uint_as_float(static_cast<uint32_t>(v[e]));
  }
}

// Coherent reads of mass words through a buffer resource over the row's
// words: the cache policy (sc1) of the device-scope relaxed atomic loads,
// 16 bytes (two adjacent heads) or 8.  Each 8-byte word was stored whole, so
// each half of a 16-byte read is one word as it was written.  Reads past the
// resource's range return zeros (no tag), so they need no bounds test.
constexpr int kCoherentPolicy = 16;
template <int HP>
struct MassRead {  // HP words, lo / hi halves
  uint32_t w[2 * HP];
};
template <int HP>
__device__ __forceinline__ MassRead<HP> coherent_words(score::SRsrc r, int word) {
  MassRead<HP> m;
  if constexpr (HP == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, word * static_cast<int>(sizeof(uint64_t)), 0,
                                                         kCoherentPolicy);
#pragma unroll
    for (int i = 0; i < 4; ++i) m.w[i] = v[i];
  } else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, word * static_cast<int>(sizeof(uint64_t)), 0,
                                                        kCoherentPolicy);
    m.w[0] = v[0];
    m.w[1] = v[1];
  }
  return m;
}
template <int HP>
__device__ __forceinline__ uint64_t word_of(const MassRead<HP>& m, int i) {
  return (static_cast<uint64_t>(m.w[2 * i + 1]) << 32) | m.w[2 * i];
}

// Without a supplied LSE: KV group g of row b, what lse_finalize_kernel does
// for it (the same merge and sums, so the same bits), from the row's mass
// words once each carries `tag`: the group's LSEs, written to lse_out, then
// each chunk's share of the group, stored as the row's tagged partial for
// its selector.  Every round issues all of its reads before it waits for
// any (reads under a per-word branch each waited for the one before).
template <int HP>
__device__ __forceinline__ void group_lse_pass(const FusedArgs& f, score::SRsrc r, const score::LseLayout& l,
                                               int C, int h0, uint32_t tag, score::LseAcc& acc) {
  using namespace score;
  const int hq = f.s.Hq;
  const int past = C * hq;  // a word index past the resource: its read returns zeros without a memory access
  for (int c0 = l.j; c0 < C; c0 += kLseLoads * l.tpp) {
    float mass[kLseLoads][HP];  // the masses of the words that carried the tag
    uint32_t missing = 0u;      // words of this round without the tag yet
#pragma unroll
    for (int u = 0; u < kLseLoads; ++u) {
#pragma unroll
      for (int i = 0; i < HP; ++i) mass[u][i] = -INFINITY;
      if (c0 + u * l.tpp < C) missing |= 1u << u;
    }
    for (uint32_t spin = 0;; ++spin) {
      // A retry reads only the words still missing (the others read past
      // the resource): polling groups that reread whole rounds slowed the
      // scoring stream that shares the memory channels.
      MassRead<HP> n[kLseLoads];
#pragma unroll
      for (int u = 0; u < kLseLoads; ++u) {
        n[u] = coherent_words<HP>(r, (missing >> u) & 1u ? (c0 + u * l.tpp) * hq + h0 : past);
      }
#pragma unroll
      for (int u = 0; u < kLseLoads; ++u) {
        bool tagged = (missing >> u) & 1u;
#pragma unroll
        for (int i = 0; i < HP; ++i) tagged = tagged && n[u].w[2 * i + 1] == tag;
#pragma unroll
        for (int i = 0; i < HP; ++i) mass[u][i] = tagged ? __uint_as_float(n[u].w[2 * i]) : mass[u][i];
        if (tagged) missing &= ~(1u << u);
      }
      if (missing == 0u) break;
      if (spin >= kSpinLimit ||
          (spin % kStatusEvery == kStatusEvery - 1 && coherent_load(f.header + kLaunchStatus) != 0u)) {
        raise_status(f.header, kStatusPartials);
        break;
      }
      __builtin_amdgcn_s_sleep(kSleep);
    }
#pragma unroll
    for (int u = 0; u < kLseLoads; ++u) {
      add_term(acc.m0, acc.z0, mass[u][0]);
      if constexpr (HP == 2) add_term(acc.m1, acc.z1, mass[u][HP - 1]);
    }
  }
}

// Each chunk's share of group g: GM >= G heads per chunk, 16 reads in
// flight per thread (2 * kLseLoads / GM chunks per thread and round).
template <int HP, int GM>
__device__ __forceinline__ void group_shares(const FusedArgs& f, score::SRsrc r, int b, int g, int C, uint32_t tag,
                                             const float* s_lse2) {
  using namespace score;
  constexpr int kChunks = 2 * kLseLoads / GM;
  constexpr int kReads = GM / HP;
  const int G = f.s.G, hq = f.s.Hq, hkv = f.s.Hkv, tid = threadIdx.x;
  uint64_t* part = f.s.tagged + static_cast<int64_t>(b) * f.s.max_chunks * hkv + g;
  for (int c0 = tid; c0 < C; c0 += kChunks * kThreads) {
    MassRead<HP> v[kChunks][kReads];
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
#pragma unroll
      for (int e = 0; e < kReads; ++e) v[k][e] = coherent_words<HP>(r, (c0 + k * kThreads) * hq + g * G + e * HP);
    }
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
      const int c = c0 + k * kThreads;
      float sum = 0.f;
#pragma unroll
      for (int h = 0; h < GM; ++h) {
        sum = h < G ? add_share(sum, __uint_as_float(v[k][h / HP].w[2 * (h % HP)]), s_lse2[h]) : sum;
      }
      if (c < C) {
        coherent_store(part + static_cast<int64_t>(c) * hkv, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(sum));
      }
    }
  }
}

template <int HP>
__device__ __forceinline__ void group_task_hp(const FusedArgs& f, score::SRsrc r, const score::LseLayout& l, int b,
                                              int g, int C, uint32_t tag, float (*s_m)[kThreads],
                                              float (*s_z)[kThreads], float* s_lse2) {
  using namespace score;
  const int G = f.s.G, tid = threadIdx.x;
  LseAcc acc;
  if (l.ph < l.P) group_lse_pass<HP>(f, r, l, C, g * G + HP * l.ph, tag, acc);
  const float lse = lse_finish(l, acc, G, s_m, s_z);
  if (tid < G) {
    f.lse_out[static_cast<int64_t>(b) * f.lse_out_stride + g * G + tid] = lse;
    s_lse2[tid] = lse_base2(lse);
  }
  __syncthreads();
  // Every word of the group was read with its tag above.
  if (G <= 8) {
    group_shares<HP, 8>(f, r, b, g, C, tag, s_lse2);
  } else {
    group_shares<HP, kMaxGroup>(f, r, b, g, C, tag, s_lse2);
  }
}

// s_m / s_z: LDS lent for the merge; s_lse2: G floats.
__device__ __forceinline__ void lse_group_task(const FusedArgs& f, int b, int g, uint32_t tag,
                                               float (*s_m)[kThreads], float (*s_z)[kThreads], float* s_lse2) {
  using namespace score;
  const ScoreArgs& sa = f.s;
  const RowDesc d = row_desc(sa.src, b);
  const int C = d.active ? (d.len + sa.chunk - 1) / sa.chunk : 0;
  if (C == 0) return;  // workgroup-uniform: a row with nothing scored
  const int G = sa.G, hq = sa.Hq;
  const uint64_t* words = sa.mw + static_cast<int64_t>(b) * sa.max_chunks * hq;
  const SRsrc r = srsrc(words, C * hq * static_cast<int>(sizeof(uint64_t)));
  // The group's word of the newest chunk and last head: written in the row's
  // last round of units.
  wait_sentinel(words + static_cast<int64_t>(C - 1) * hq + g * G + G - 1, tag, f.header);
  const LseLayout l = lse_layout(G, f.lse_wide, threadIdx.x);
  if (l.hp == 2) {
    group_task_hp<2>(f, r, l, b, g, C, tag, s_m, s_z, s_lse2);
  } else {
    group_task_hp<1>(f, r, l, b, g, C, tag, s_m, s_z, s_lse2);
  }
}

// Selection and plan of batch row b (the select_plan_kernel steps, with the
// partials polled from the workspace), then the row's flag.
__device__ __forceinline__ void select_row(const FusedArgs& f, int b, uint32_t tag,
                                           select::SelectShared<kFusedKeys>& sh) {
  using namespace select;
  const SelectArgs& a = f.p;
  const int tid = threadIdx.x;
  const RowDesc d = row_desc(a.src, b);
  const int slot = a.slots[b];
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  // Made scalar (waited for) here: they are used only after the selection's
  // stores, where waiting for their loads would wait for those stores too.
  const int committed = __builtin_amdgcn_readfirstlane(committed_of(a.committed_lens, a.src, b));
  const int stored_count = __builtin_amdgcn_readfirstlane(slot_ok ? a.counts[slot] : 0);
  uint32_t gen = __builtin_amdgcn_readfirstlane((f.rec != nullptr && slot_ok) ? static_cast<uint32_t>(f.gen[slot]) : 0u);
  // The previous row's plan columns are read from sh.ids up to its end.
  lds_barrier();
  if (f.expire && tid == 0) raise_status(f.header, kStatusPartials);
  int n_sel = -1;
  if (d.active && slot_ok) {
    const int C = (d.len + a.chunk - 1) / a.chunk;
    const int K = a.budget / a.chunk;
    if (C <= K) {
      for (int i = tid; i < C; i += kThreads) sh.ids[i] = i;
      n_sel = C;
    }
    float* row_scores = a.scores + static_cast<int64_t>(b) * a.score_stride;
    const int N = C - 1;
    const bool in_lds = C > K && N <= kFusedKeys;
    const uint64_t* part = f.s.tagged + static_cast<int64_t>(b) * a.max_chunks * a.hkv;
    const int per_poll = kPollLoads / a.hkv;  // chunks per thread and poll
    uint32_t kmin = ~0u, kmax = 0u;           // bounds of this thread's candidate keys
    for (int base = 0; base < C; base += per_poll * kThreads) {
      float sum[kPollLoads];
      poll_chunk_sums(part, base, C, a.hkv, tag, f.header, sum);
#pragma unroll
      for (int u = 0; u < kPollLoads; ++u) {
        const int i = base + u * kThreads + tid;
        if (u < per_poll && i < C) {
          const float v = chunk_score(sum[u], a.chunk, d.len, i, a.hq);
          row_scores[i] = v;
          if (i < N) {
            const uint32_t key = order_key(v);
            kmin = min(kmin, key);
            kmax = max(kmax, key);
            if (in_lds) sh.keys[i] = key;
          }
        }
      }
    }
    if (in_lds) {
      lds_barrier();
    } else {
      __syncthreads();  // keys are read back from the score row in global memory
    }
    if (C > K) {
      select_top(sh, N, K, [&](int q) -> U4 {
        if (in_lds) return *reinterpret_cast<const U4*>(&sh.keys[4 * q]);
        U4 k4;
#pragma unroll
        for (int j = 0; j < 4; ++j) k4[j] = order_key(row_scores[min(4 * q + j, N - 1)]);
        return k4;
      }, kmin, kmax);
      n_sel = K;
    }
    lds_barrier();
    int32_t* out = a.ids + static_cast<int64_t>(slot) * a.ids_stride;
    for (int j = tid; j < n_sel; j += kThreads) out[j] = sh.ids[j];
    ++gen;
    if (tid == 0) {
      a.counts[slot] = n_sel;
      if (f.rec != nullptr) f.gen[slot] = static_cast<int32_t>(gen);
    }
  }
  uint64_t* tagged = f.plans + static_cast<int64_t>(b) * kPlanCols;
  if (f.rec != nullptr && tid == 0) coherent_store(tagged + kGenCol, (static_cast<uint64_t>(tag) << 32) | gen);
  if (slot_ok) {
    write_plan_row(a, b, slot, committed, n_sel, stored_count, sh, tagged, tag);
  } else {
    int64_t* prow = a.plan + static_cast<int64_t>(b) * a.plan_width;
    for (int j = tid; j < a.plan_width; j += kThreads) {
      prow[j] = 0;
      coherent_store(tagged + j, static_cast<uint64_t>(tag) << 32);
    }
  }
}

// A plan row as a gathering wave sees it: the fields, wave-uniform, and
// the columns, lane l holding columns l (lo) and 64 + l (hi).
struct PlanView {
  int64_t slot, len, tail_start, prefix_len, drop;
  int64_t hist_len;  // the plan's history length (len is it clipped to the cos/sin rows)
  uint32_t lo, hi;
  uint32_t gen;  // the slot's selection generation (with gather records)
};

// Polls row r's tagged plan until every column carries the tag, at most
// `spins` polls (then returns false).
__device__ __forceinline__ bool poll_plan(const FusedArgs& f, int r, uint32_t tag, uint32_t spins, PlanView& v) {
  const gather::GatherArgs& ga = f.g;
  const int lane = threadIdx.x & 63;
  const uint64_t* row = f.plans + static_cast<int64_t>(r) * kPlanCols;
  const bool has_lo = lane < ga.plan_width;
  const bool has_hi = lane + 64 < ga.plan_width || (f.rec != nullptr && lane + 64 == kGenCol);
  for (uint32_t spin = 0; spin < spins; ++spin) {
    const uint64_t a = has_lo ? coherent_load(row + lane) : static_cast<uint64_t>(tag) << 32;
    const uint64_t b = has_hi ? coherent_load(row + 64 + lane) : static_cast<uint64_t>(tag) << 32;
    if (__ballot(static_cast<uint32_t>(a >> 32) != tag || static_cast<uint32_t>(b >> 32) != tag) == 0) {
      v.lo = static_cast<uint32_t>(a);
      v.hi = static_cast<uint32_t>(b);
      v.slot = static_cast<int32_t>(__builtin_amdgcn_readlane(v.lo, 0));
      v.hist_len = static_cast<int32_t>(__builtin_amdgcn_readlane(v.lo, 1));
      v.len = min(v.hist_len, static_cast<int64_t>(ga.pos_limit));
      v.tail_start = static_cast<int32_t>(__builtin_amdgcn_readlane(v.lo, 2));
      v.prefix_len = static_cast<int32_t>(__builtin_amdgcn_readlane(v.lo, 3));
      v.drop = static_cast<int32_t>(__builtin_amdgcn_readlane(v.lo, 4));
      v.gen = static_cast<uint32_t>(__builtin_amdgcn_readlane(v.hi, kGenCol - 64));
      if (v.slot < 0 || v.slot >= ga.num_slots) v.len = 0;
      return true;
    }
    __builtin_amdgcn_s_sleep(kSleep);
  }
  return false;
}

// Gather task t (local positions t * ppw ...) of the row in `v`.
template <int DT, bool NEOX>
__device__ __forceinline__ void run_task(const gather::GatherArgs& ga, const gather::GatherLane& L,
                                         const PlanView& v, int t) {
  const int ppw = 64 / ga.lanes_per_row;
  gather::gather_task<DT, NEOX, kGatherHeads>(
      ga, L, t * ppw, v.slot, v.len, v.tail_start, v.prefix_len, v.drop, [&](int64_t c) {
        // Chunk id column 5 + c sits in lane (5 + c) % 64 of lo or hi.
        const int col = static_cast<int>(5 + c);
        const int lo = __builtin_amdgcn_ds_bpermute((col & 63) << 2, static_cast<int>(v.lo));
        const int hi = __builtin_amdgcn_ds_bpermute((col & 63) << 2, static_cast<int>(v.hi));
        return static_cast<int64_t>(col < 64 ? lo : hi);
      });
}

// Gather record of task t of the row whose slot is `slot` (0 without records
// or for a slot out of range), requested before the row's plan arrives.
__device__ __forceinline__ uint64_t task_record(const FusedArgs& f, int slot, int t) {
  return (f.rec != nullptr && slot >= 0 && slot < f.g.num_slots) ? f.rec[static_cast<int64_t>(slot) * f.rec_stride + t]
                                                                  : 0u;
}

// Gather task t of the row in `v`, keeping its gather record: a task whose
// record shows the working cache already holds its bytes is left out, and
// with prefix_only so is every task not wholly in the history prefix.
template <int DT, bool NEOX>
__device__ __forceinline__ void gather_recorded(const FusedArgs& f, const gather::GatherLane& L, const PlanView& v,
                                                int r, int t, uint64_t have) {
  const int ppw = 64 / f.g.lanes_per_row;
  const int p0 = t * ppw;
  // Before the draft's prefill (prefix_only), only a task whose raw rows all
  // precede the rows that prefill rewrites is moved (and recorded).
  const bool early_ok =
      !f.prefix_only || gather::sources_final(p0, ppw, v.tail_start, v.prefix_len, first_rewritten(f.p.src, r));
  const uint64_t want =
      p0 + ppw <= v.len && early_ok
          ? gather::history_record(p0, ppw, v.hist_len, v.tail_start, v.prefix_len, v.drop, v.gen)
          : 0u;
  bool move = !f.prefix_only || want != 0u;
  if (f.rec != nullptr && v.slot >= 0 && v.slot < f.g.num_slots) {
    have = static_cast<uint64_t>(uniform64(static_cast<int64_t>(have)));
    if (want != 0u && have == want) move = false;
    if ((threadIdx.x & 63) == 0 && have != want) f.rec[v.slot * f.rec_stride + t] = want;
  }
  if (move) run_task<DT, NEOX>(f.g, L, v, t);
}

// A scoring wave's gather tasks: task numbers gw, gw + tw, ... of the
// row-major numbering in task_prefix (exclusive prefix of the rows' task
// counts).  Each waits for its row's plan at most kOwnerSpins polls; a task
// whose plan did not come in time is marked skipped, and the launch's skip
// word is set, for the last workgroup to finish.  Both writes are
// read-modify-writes the wave waits for, so they are in memory before its
// workgroup counts itself done.
template <int DT, bool NEOX>
__device__ __forceinline__ void gather_owned(const FusedArgs& f, const int* task_prefix, const int* row_slot, int gw,
                                             int tw, uint32_t tag) {
  const gather::GatherArgs& ga = f.g;
  const int rows = f.p.batch;
  const gather::GatherLane L = gather::gather_lane<DT, NEOX>(ga);
  const int total = task_prefix[rows];
  int cur = -1, hint = 0;
  bool published = false;
  PlanView v{};
  for (int task = gw; task < total; task += tw) {
    int lo = hint, hi = rows - 1;  // task numbers grow along the wave's list
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (task_prefix[mid] <= task) lo = mid; else hi = mid - 1;
    }
    hint = lo;
    const int r = __builtin_amdgcn_readfirstlane(lo);
    const int t = __builtin_amdgcn_readfirstlane(task - task_prefix[r]);
    const uint64_t have = task_record(f, row_slot[r], t);
    if (r != cur) {
      cur = r;
      published = poll_plan(f, r, tag, f.owner_spins, v);
    }
    if (published) {
      gather_recorded<DT, NEOX>(f, L, v, r, t, have);
    } else if ((threadIdx.x & 63) == 0) {
      __hip_atomic_exchange(f.state + static_cast<int64_t>(r) * f.task_cap + t, tag | kSkipped, __ATOMIC_ACQUIRE,
                            __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_exchange(f.header + kSkips, tag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The gather tasks their scoring waves skipped, done by the last workgroup
// to finish: every other workgroup has counted itself done, so every plan is
// published and every skip mark is in memory.  Each wave checks 64 tasks of
// a row at a time.  A bit a wait raises here goes straight to the owner's
// words, since the launch's status word has already been handed over.
template <int DT, bool NEOX>
__device__ __forceinline__ void redo_skipped(const FusedArgs& f, const int* task_prefix, uint32_t tag) {
  const int lane = threadIdx.x & 63;
  const gather::GatherLane L = gather::gather_lane<DT, NEOX>(f.g);
  for (int b = 0; b < f.p.batch; ++b) {
    const int tasks = task_prefix[b + 1] - task_prefix[b];
    const uint32_t* st = f.state + static_cast<int64_t>(b) * f.task_cap;
    bool have_plan = false, failed = false;  // a plan that never came is waited for once per row
    PlanView v{};
    for (int t0 = static_cast<int>(threadIdx.x >> 6) * 64; t0 < tasks && !failed; t0 += kThreads) {
      const int t = t0 + lane;
      const uint32_t s = t < tasks ? coherent_load(st + t) : 0u;
      uint64_t skipped = __ballot(s == (tag | kSkipped));
      while (skipped != 0) {
        const int k = __builtin_ctzll(skipped);
        skipped &= skipped - 1;
        if (!have_plan) {
          have_plan = poll_plan(f, b, tag, kSpinLimit, v);
          if (!have_plan) {
            if (lane == 0) {
              __hip_atomic_fetch_or(f.header + kStatus, kStatusTasks, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              if (f.status_out != nullptr) {
                __hip_atomic_fetch_or(f.status_out, kStatusTasks, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              }
            }
            failed = true;
            break;
          }
        }
        gather_recorded<DT, NEOX>(f, L, v, b, t0 + k, task_record(f, static_cast<int>(v.slot), t0 + k));
      }
    }
  }
}

struct WorkShared {
  int unit_prefix[kFusedRows + 1];
  int len[kFusedRows];
  int qrow[kFusedRows];
  int scratch[4];
};

template <int DT, int STEPS, bool NEOX, int PAGE, bool LSEFREE>
__global__ __launch_bounds__(kThreads, 3) void fused_step_kernel(FusedArgs f) {
  constexpr int KB = STEPS <= 2 ? 2 : 1;  // chunk_score_kernel's batch shape (4 KB) for head_dim <= 128
  __shared__ union {
    select::SelectShared<kFusedKeys> sel;
    WorkShared w;
  } lds;
  __shared__ int s_task_prefix[kFusedRows + 1];
  __shared__ int s_slot[kFusedRows];  // each row's slot (gather records are per slot)
  __shared__ int s_scratch[4];
  __shared__ uint32_t s_tag;
  __shared__ uint32_t s_last;
  __shared__ float s_lse2[LSEFREE ? score::kMaxGroup : 1];  // a group's exponent bases (no LSE supplied)

  const int rows = f.p.batch;
  const gather::GatherArgs& ga = f.g;
  if (threadIdx.x == 0) {
    const uint32_t t = (coherent_load(f.header + kEpoch) + 1u) & ~kSkipped;
    s_tag = t == 0u ? 1u : t;
  }
  // One round of row loads serves both work lists (rows <= kThreads: thread
  // r loads row r).  Gather tasks of row r: its history length is at most
  // min(committed - 1, pos_limit) (plan construction bounds it by the
  // history end), so the task list is known before any plan exists.  The
  // scoring workgroups also take row r's scored length and query row.
  const int ppw = 64 / ga.lanes_per_row;
  const int first_selector = static_cast<int>(gridDim.x) - f.selectors;
  const bool selector = static_cast<int>(blockIdx.x) >= first_selector;
  const int tr = static_cast<int>(threadIdx.x);
  int row_tasks = 0;
  RowDesc own{0, 0, 0};
  if (tr < rows) {
    const int slot = f.p.slots[tr];
    s_slot[tr] = slot;
    const bool gathered = (ga.row_active == nullptr || ga.row_active[tr] != 0) && slot >= 0 && slot < ga.num_slots;
    const int committed = committed_of(f.p.committed_lens, f.p.src, tr);
    if (!selector) own = row_desc(f.s.src, tr);
    row_tasks = gathered ? (min(max(committed - 1, 0), ga.pos_limit) + ppw - 1) / ppw : 0;
  }
  build_row_prefix(rows, s_task_prefix, s_scratch, [&](int) { return row_tasks; });
  const uint32_t tag = s_tag;

  if (selector) {
    const int s = static_cast<int>(blockIdx.x) - first_selector;
    if constexpr (LSEFREE) {
      // The first group_selectors workgroups do the KV groups' shares, one
      // per (row slot, group); the row selectors above them (higher indices:
      // every wait is on lower-indexed workgroups) select as with an LSE.
      const int hkv = f.s.Hkv;
      const int gs = f.group_selectors;
      if (s < gs) {
        float(*s_m)[kThreads] = reinterpret_cast<float(*)[kThreads]>(&lds.sel.keys[0]);
        for (int b = s / hkv; b < rows; b += gs / hkv) {
          lds_barrier();  // the merge borrows the key area between rows
          lse_group_task(f, b, s % hkv, tag, s_m, s_m + 2, s_lse2);
        }
      } else {
        for (int b = s - gs; b < rows; b += f.selectors - gs) select_row(f, b, tag, lds.sel);
      }
    } else {
      for (int b = s; b < rows; b += f.selectors) select_row(f, b, tag, lds.sel);
    }
  } else {
    WorkShared& w = lds.w;
    const score::ScoreArgs& sa = f.s;
    if (tr < rows) {
      w.len[tr] = own.active ? own.len : 0;
      w.qrow[tr] = static_cast<int>(own.qrow);
    }
    __syncthreads();
    build_row_prefix(rows, w.unit_prefix, w.scratch, [&](int r) { return (w.len[r] + sa.U - 1) / sa.U * sa.Hkv; });
    const int gw = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kWaves +
                                                  static_cast<int>(threadIdx.x >> 6));
    const int tw = first_selector * kWaves;
    score::score_stream<DT, STEPS, KB, false, PAGE, true, LSEFREE>(sa, w.unit_prefix, w.len, w.qrow,
                                                                   w.unit_prefix[rows], gw, tw, tag);
    gather_owned<DT, NEOX>(f, s_task_prefix, s_slot, gw, tw, tag);
  }

  // The last workgroup to finish hands this launch's status bits to the
  // owner's word, clears them for the next launch, redoes the gather tasks
  // their scoring waves skipped, and publishes the tag as the epoch.  Every
  // raise and skip mark of a workgroup has returned before that workgroup's
  // count (the barrier below orders them), so the last count comes after all
  // of them.  The atomics are relaxed: a release here would write back the
  // XCD's L2 in every workgroup.
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(f.header + kDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t last = 0u;
    if (prev == gridDim.x - 1) {
      const uint32_t bits =
          __hip_atomic_exchange(f.header + kLaunchStatus, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t skips = __hip_atomic_exchange(f.header + kSkips, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (bits != 0u) {
        __hip_atomic_fetch_or(f.header + kStatus, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (f.status_out != nullptr) {
          __hip_atomic_fetch_or(f.status_out, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      last = skips == tag ? 3u : 1u;
      if (last == 1u) {
        coherent_store(f.header + kDone, 0u);
        coherent_store(f.header + kEpoch, tag);
      }
    }
    s_last = last;
  }
  __syncthreads();
  if (s_last == 3u) {
    redo_skipped<DT, NEOX>(f, s_task_prefix, tag);
    if (threadIdx.x == 0) {
      coherent_store(f.header + kDone, 0u);
      coherent_store(f.header + kEpoch, tag);
    }
  }
}

size_t plans_bytes(int rows) { return static_cast<size_t>(rows) * kPlanCols * sizeof(uint64_t); }
int task_cap(int token_budget) { return (token_budget + kMinTaskPositions - 1) / kMinTaskPositions; }
size_t state_bytes(int rows, int token_budget) {
  return (static_cast<size_t>(rows) * task_cap(token_budget) * sizeof(uint32_t) + kLine - 1) / kLine * kLine;
}

// Grid: the workgroups that fit on the device at once (occupancy from the
// runtime), fewer when the work is smaller; the last `selectors` select.
template <auto Kernel>
int launch_fused(hipStream_t stream, const FusedArgs& f, int64_t upper_units, int64_t upper_tasks, bool& launched) {
  static int per_cu = -1;
  if (per_cu < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, Kernel, kThreads, 0) != hipSuccess) n = 0;
    per_cu = n;
  }
  const int64_t resident = static_cast<int64_t>(per_cu) * device_cu_count();
  if (resident < f.selectors + 1) return clear_error();  // does not fit: the chain runs instead
  const int64_t work_wgs = std::max<int64_t>(
      1, std::max((upper_units + kWaves - 1) / kWaves, (upper_tasks + kWaves - 1) / kWaves));
  const int grid = static_cast<int>(f.selectors + std::min(resident - f.selectors, work_wgs));
  Kernel<<<grid, kThreads, 0, stream>>>(f);
  const int rc = check_launch("fused retrieval step");
  launched = rc == DS_OK;
  return rc;
}

template <int DT, int PAGE, bool LSEFREE>
int launch_page(hipStream_t stream, const FusedArgs& f, int steps, bool neox, int64_t upper_units,
                int64_t upper_tasks, bool& launched) {
  if (steps == 4) {
    if (neox) {
      return launch_fused<fused_step_kernel<DT, 4, true, PAGE, LSEFREE>>(stream, f, upper_units, upper_tasks,
                                                                         launched);
    }
    return launch_fused<fused_step_kernel<DT, 4, false, PAGE, LSEFREE>>(stream, f, upper_units, upper_tasks,
                                                                        launched);
  }
  if (neox) {
    return launch_fused<fused_step_kernel<DT, 2, true, PAGE, LSEFREE>>(stream, f, upper_units, upper_tasks, launched);
  }
  return launch_fused<fused_step_kernel<DT, 2, false, PAGE, LSEFREE>>(stream, f, upper_units, upper_tasks, launched);
}

template <int DT, bool LSEFREE>
int launch_lse(hipStream_t stream, const FusedArgs& f, int steps, bool neox, int page_mode, int64_t upper_units,
               int64_t upper_tasks, bool& launched) {
  if (page_mode == score::PAGE_POW2) {
    return launch_page<DT, score::PAGE_POW2, LSEFREE>(stream, f, steps, neox, upper_units, upper_tasks, launched);
  }
  return launch_page<DT, score::PAGE_UNIFORM, LSEFREE>(stream, f, steps, neox, upper_units, upper_tasks, launched);
}

template <int DT>
int launch_dt(hipStream_t stream, const FusedArgs& f, int steps, bool neox, int page_mode, bool lse_free,
              int64_t upper_units, int64_t upper_tasks, bool& launched) {
  if (lse_free) return launch_lse<DT, true>(stream, f, steps, neox, page_mode, upper_units, upper_tasks, launched);
  return launch_lse<DT, false>(stream, f, steps, neox, page_mode, upper_units, upper_tasks, launched);
}

}  // namespace

size_t fused_workspace_bytes(int rows, int max_chunks, int num_kv_heads, int token_budget) {
  if (rows <= 0 || max_chunks <= 0 || num_kv_heads <= 0 || token_budget <= 0) return 0;
  return kHeaderWords * sizeof(uint32_t) + plans_bytes(rows) + state_bytes(rows, token_budget) +
         static_cast<size_t>(rows) * max_chunks * num_kv_heads * sizeof(uint64_t);
}

// Runs the whole step as one launch when the descriptor fits the fused
// kernel; `launched` stays false (and nothing is launched) otherwise.
int launch_fused_step(hipStream_t stream, const ds_step_desc* d, const RowSource& src, uint32_t* status_out,
                      bool& launched) {
  launched = false;
  const bool prefix = d->stages == (DS_STAGE_SCORE | DS_STAGE_SELECT | DS_STAGE_PREFIX);
  if (d->workspace == nullptr || (d->stages != DS_STAGE_ALL && !prefix)) return clear_error();
  // Without a supplied LSE the selectors merge each row's mass words, which
  // live in the caller's lse_partials ([batch_rows, max_chunks, Hq] 64-bit
  // words); a row's words are read through 32-bit byte offsets, which the
  // reads of a round may overrun by kLseLoads * kThreads chunks (they return
  // zeros).
  const bool lse_free = d->lse == nullptr;
  if (lse_free && (d->lse_partials == nullptr || d->lse_out == nullptr || d->lse_out_stride < d->num_q_heads ||
                   (static_cast<int64_t>(d->max_chunks) + score::kLseLoads * kThreads) * d->num_q_heads *
                           static_cast<int64_t>(sizeof(uint64_t)) >
                       INT32_MAX)) {
    return clear_error();
  }
  const size_t need = fused_workspace_bytes(d->batch_rows, d->max_chunks, d->num_kv_heads, d->token_budget);
  DS_REQUIRE(need > 0 && d->workspace_bytes >= need,
             "step workspace too small: need %zu bytes for %d rows, %d chunks, %d KV heads, token budget %d", need,
             d->batch_rows, d->max_chunks, d->num_kv_heads, d->token_budget);
  DS_REQUIRE((reinterpret_cast<uintptr_t>(d->workspace) & 63u) == 0, "step workspace must be 64-byte aligned");

  FusedArgs f{};
  int64_t upper_units = 0;
  int page_mode = score::PAGE_LANE;
  int rc = make_score_args(f.s, upper_units, page_mode, d->dtype, d->query, d->q_stride, d->key_cache,
                           d->k_block_stride, d->k_token_stride, d->k_head_stride, d->lse, d->lse_token_stride,
                           d->lse_head_stride, d->block_table, d->bt_stride, src, d->batch_rows, d->num_q_heads,
                           d->num_kv_heads, d->head_dim, d->block_size, d->chunk_size, d->max_chunks, d->scale,
                           DS_HEAD_MEAN, d->score_partials, nullptr, 0, 0, SIZE_MAX,
                           lse_free ? reinterpret_cast<uint64_t*>(d->lse_partials) : nullptr);
  if (rc != DS_OK) return rc;
  rc = make_select_args(f.p, d->scores, d->max_chunks, d->score_partials, d->max_chunks, d->num_kv_heads,
                        d->num_q_heads, src, d->batch_rows, d->chunk_size, d->history_budget, 1, 1, d->sel_ids,
                        d->sel_stride, d->sel_count, d->slots, d->num_slots, d->committed_lens, d->plan,
                        d->plan_width, d->working_lens, d->recent_window);
  if (rc != DS_OK) return rc;
  bool vec = false;
  int scalar_grid = 0;
  rc = make_gather_args(f.g, vec, scalar_grid, d->kv_dtype, d->raw_key, d->raw_value, d->working_key,
                        d->working_value, d->plan, d->batch_rows, d->plan_width, d->cos_sin, d->cs_stride,
                        d->cs_rows, d->num_slots, d->max_model_len, d->draft_heads, d->draft_head_dim,
                        d->token_budget, d->chunk_size, d->rotary_dim, d->is_neox_style, d->history_budget,
                        d->row_active, true);
  if (rc != DS_OK) return rc;

  // Shapes the fused kernel is built for; everything else runs the chain.
  const int steps = d->head_dim / 32;
  const bool fits = d->dtype == d->kv_dtype && (d->dtype == DS_BF16 || d->dtype == DS_FP16) &&
                    (d->head_dim == 64 || d->head_dim == 128) && d->num_kv_heads <= kMaxHkv &&
                    d->batch_rows >= kMinFusedRows && d->batch_rows <= kFusedRows && page_mode != score::PAGE_LANE && vec &&
                    scalar_grid > 0 && d->slots != nullptr && d->plan_width <= kPlanCols &&
                    64 / f.g.lanes_per_row >= kMinTaskPositions &&
                    (d->gather_rec == nullptr || d->plan_width < kGenCol + 1);
  if (!fits) return clear_error();

  char* ws = static_cast<char*>(d->workspace);
  f.header = reinterpret_cast<uint32_t*>(ws);
  ws += kHeaderWords * sizeof(uint32_t);
  f.plans = reinterpret_cast<uint64_t*>(ws);
  ws += plans_bytes(d->batch_rows);
  f.state = reinterpret_cast<uint32_t*>(ws);
  f.task_cap = task_cap(d->token_budget);
  ws += state_bytes(d->batch_rows, d->token_budget);
  f.s.tagged = reinterpret_cast<uint64_t*>(ws);
  f.selectors = std::min(d->batch_rows, kSelectors);
  f.owner_spins = (d->flags & DS_STEP_SELECTORS_GATHER) != 0 ? 0u : kOwnerSpins;
  f.expire = (d->flags & DS_STEP_EXPIRE_WAITS) != 0 ? 1 : 0;
  f.status_out = status_out;
  if (d->gather_rec != nullptr) {
    f.gen = d->sel_gen;
    f.rec = d->gather_rec;
    f.rec_stride = d->rec_stride;
  }
  f.prefix_only = prefix ? 1 : 0;
  if (lse_free) {
    // kGroupSelectors / Hkv row slots of Hkv group workgroups, taking rows
    // s, s + slots, ... (rows finish roughly in order), below the row
    // selectors.
    f.group_selectors =
        std::min(d->batch_rows, std::max(1, kGroupSelectors / d->num_kv_heads)) * d->num_kv_heads;
    f.selectors += f.group_selectors;
    f.lse_out = d->lse_out;
    f.lse_out_stride = d->lse_out_stride;
    f.lse_wide = score::lse_words_wide(d->lse_partials);
  }
  if (prefix) f.p.working_lens = nullptr;  // the compact prefill sets them
  const int ppw = 64 / f.g.lanes_per_row;
  const int64_t upper_tasks = static_cast<int64_t>(d->batch_rows) * ((f.g.pos_limit + ppw - 1) / ppw);
  const bool neox = d->is_neox_style != 0;
  if (d->dtype == DS_BF16) {
    return launch_dt<DS_BF16>(stream, f, steps, neox, page_mode, lse_free, upper_units, upper_tasks, launched);
  }
  return launch_dt<DS_FP16>(stream, f, steps, neox, page_mode, lse_free, upper_units, upper_tasks, launched);
}

}  // namespace ds355

extern "C" size_t ds_step_workspace_bytes(int batch_rows, int max_chunks, int num_kv_heads, int token_budget) {
  return ds355::fused_workspace_bytes(batch_rows, max_chunks, num_kv_heads, token_budget);
}
