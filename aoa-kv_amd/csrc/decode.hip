// AOA-KV decode path on gfx950: page scoring, per-head top-k and split-K
// sparse decode attention over the selected pages.
//
// Replaces, with the simulation's semantics (filter_util.py:269-407,
// 968-1018; quest_attention.py:265-356):
//   MaxPossibleSampleWithPagedKVCacheKernel  decode_attn.cuh:276-443
//   decode_select_k (RAFT radix one-block)   decode_select_k.cuh:26-61
//   BatchDecodeWithPagedKVCacheKernel +      decode_attn.cuh:482-688,
//   VariableLengthMergeStates                1004-1044
//
// All three stages are HBM-bound scans / gathers.  Each wave owns four
// 16-lane rows; a row covers one 128-dim fp16 vector with 16-byte loads, so
// one wave-wide load moves 1 KB.  Cross-workgroup steps (top-k after all of
// a head's scores are written, the split-K merge) are done by the last
// workgroup to arrive at a per-head counter (arrive_last), with the data
// handed over through agent-coherent stores and loads.  Loads that feed a
// reduction are issued as a batch before any of them is consumed, so a
// handoff costs one memory round trip, not one per element.
#include "kernels.hpp"

#include <type_traits>

namespace aoakv {

constexpr int kThreads = 256;
constexpr int kEstPagesPerWave = 32;                     // 8 steps x 4 rows
constexpr int kEstPagesPerBlock = kEstPagesPerWave * 4;  // 128
// Pages per scoring item: with a GQA group of G query heads a page costs G
// bounds, so an item takes 128 / G pages (the same arithmetic per item, G
// times the items to spread over the CUs).
template <int GROUP>
constexpr uint32_t est_block_pages() {
  return (uint32_t)kEstPagesPerBlock / (uint32_t)GROUP;
}
__host__ __device__ constexpr uint32_t est_block_pages_of(uint32_t group) {
  return (uint32_t)kEstPagesPerBlock / group;
}
// Items of the scoring kernel without the fused top-k (the three-call
// path's estimate): half as large at GROUP = 1, so each CU holds more items'
// dependent page-table and metadata chains in flight (config 2: 9.0 against
// 10.6 us; a quarter as large: 9.1).  The fused kernel keeps 128 pages: its
// last item per head selects, and with twice the items that tail grew (14.1
// against 13.7 us).  The page scores do not depend on the item size.
template <int GROUP, bool FUSED>
constexpr uint32_t est_kernel_block_pages() {
  return GROUP == 1 && !FUSED ? est_block_pages<1>() / 2u : est_block_pages<GROUP>();
}
__host__ __device__ constexpr uint32_t est_kernel_block_pages_of(uint32_t group, bool fused) {
  return group == 1u && !fused ? est_block_pages_of(1u) / 2u : est_block_pages_of(group);
}
constexpr int kDecPagesPerWave = 2;
constexpr int kDecPagesPerBlock = kDecPagesPerWave * 4;  // 8
constexpr int kPartialStride = kHeadDim + 4;             // o[128], m, l, pad
constexpr int kMergeMaxChunks = 1024;                    // decode chunks per head
constexpr uint32_t kTopkMaxPages = 16384;

// ---------------------------------------------------------------- timeline
// With AOAKV_TIMELINE defined (a separate profiling build, never the shipped
// library), thread 0 of each workgroup notes the s_memrealtime counter (100
// MHz, one clock for the whole GPU) at the phase points below in LDS, and
// writes them out once, when the workgroup ends (TL_FLUSH), to its row of
// g_tl (linear workgroup index): no global access between the points, so the
// notes barely move the phases they time.  Every instrumented launch
// overwrites the rows of its workgroups; aoakv_timeline_read (end of this
// file) reads them back.  Without AOAKV_TIMELINE, TL() is empty.
enum : int {
  kTlStart = 0,        // workgroup entry
  kTlStaggerDone = 1,  // staggered start over (scoring workers, decode items)
  kTlScored0 = 2,      // scoring worker: first item's scores stored
  kTlScored1 = 3,      // ... second item's
  kTlScoresSeen = 4,   // top-k: the head's scores seen (sentinel / counter)
  kTlRowLoaded = 5,    // top-k: every score word of the row loaded
  kTlSelected = 6,     // top-k: radix select done
  kTlSelInHand = 7,    // decode item: its selection entries known
  kTlAttended = 8,     // decode item: K/V gathered and attended
  kTlPartial = 9,      // decode item: partial (o, m, l) stored
  kTlMergeLoaded = 10, // merging item: every partial loaded
  kTlOutput = 11,      // merging item: output stored (top-k workgroup: selection stored)
  kTlStaged = 12,      // top-k: keys staged, key range reduced
  kTlPass1 = 13,       // top-k: first radix pass done
  kTlXcc = 14,         // (not a time) the XCD the workgroup ran on (HW_REG_XCC_ID)
  kTlClk0 = 15,        // (core clock counter, s_memtime) at the workgroup's start
  kTlClk1 = 16,        // ... and at its end
  kTlEvents = 17
};
#ifdef AOAKV_TIMELINE
constexpr uint32_t kTlMaxWg = 4096;
__device__ unsigned long long g_tl[kTlMaxWg][kTlEvents];
__shared__ unsigned long long s_tl[kTlEvents];
#define TL(ev)                                                             \
  do {                                                                     \
    if (threadIdx.x == 0u) s_tl[ev] = __builtin_amdgcn_s_memrealtime();   \
  } while (0)
#define TL_BEGIN()                                                         \
  do {                                                                     \
    if (threadIdx.x == 0u) {                                               \
      for (int e_ = 0; e_ < kTlEvents; ++e_) s_tl[e_] = 0ull;              \
      s_tl[kTlXcc] = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (15 << 11)); \
      s_tl[kTlClk0] = __builtin_amdgcn_s_memtime();                        \
    }                                                                      \
  } while (0)
#define TL_FLUSH()                                                                         \
  do {                                                                                     \
    const uint32_t tl_wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z); \
    if (threadIdx.x == 0u && tl_wg < kTlMaxWg) {                                           \
      s_tl[kTlClk1] = __builtin_amdgcn_s_memtime();                                        \
      for (int e_ = 0; e_ < kTlEvents; ++e_) g_tl[tl_wg][e_] = s_tl[e_];                   \
    }                                                                                      \
  } while (0)
#else
#define TL(ev) \
  do {         \
  } while (0)
#define TL_BEGIN() \
  do {             \
  } while (0)
#define TL_FLUSH() \
  do {             \
  } while (0)
#endif

// ======================================================================
// block-wide helpers (256 threads = 4 waves)
// ======================================================================

// Inclusive prefix sum over the 64 lanes of a wave: DPP row_shr steps inside
// each 16-lane row, then the totals of the rows below through readlane.
__device__ inline uint32_t wave_incl_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);  // row_shr:8
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const uint32_t row = __lane_id() / kLanesPerRow;
  return v + (row > 0u ? r0 : 0u) + (row > 1u ? r1 : 0u) + (row > 2u ? r2 : 0u);
}

// min / max of a uint32 over the wave (DPP inside rows, readlane across)
template <bool MAX>
__device__ inline uint32_t wave_reduce_u32(uint32_t v) {
  auto op = [](uint32_t x, uint32_t y) { return MAX ? (x > y ? x : y) : (x < y ? x : y); };
  v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kQuadSwap1, 0xf, 0xf, true));
  v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kQuadSwap2, 0xf, 0xf, true));
  v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kRowHalfMirror, 0xf, 0xf, true));
  v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kRowMirror, 0xf, 0xf, true));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return op(op(a, b), op(c, d));
}

// ======================================================================
// top-k selection for one (sequence, kv head), one 256-thread block
// ======================================================================

// Bound on polls of a handoff word before a wait gives up (it then sets the
// error flag and goes on with stand-in data, so every wave still exits).
constexpr uint32_t kSpinLimit = 1u << 18;

// Sleeps until `ps` picoseconds of wall time have passed since t0, a reading
// of s_memrealtime: a 100 MHz counter of its own, so the wait does not scale
// with the core clock (1.3-2.6 GHz with load and temperature).  The counter
// is read a few times per wait, not polled: between reads the wave sleeps
// for a bound on the time left (one `s_sleep 1` lasts 64 core cycles, at
// most 5 ticks at 1.3 GHz), so each read finds at most the time left and
// the reads converge on the end.  Polling a clock (s_memrealtime or
// s_memtime) in every waiting wave slowed the whole layer by 0.4-1 us.
__device__ inline void sleep_until(uint64_t t0, uint64_t ps) {
  const uint64_t end = t0 + ps / 10000u;
  for (uint64_t now = __builtin_amdgcn_s_memrealtime(); now < end;
       now = __builtin_amdgcn_s_memrealtime()) {
    for (uint32_t n = (uint32_t)((end - now) / 5u) + 1u; n != 0u; --n) __builtin_amdgcn_s_sleep(1);
  }
}

// Polls an agent-coherent handoff word until it is written (non-zero);
// returns the value - 1, or 0 after kSpinLimit polls with *error set.
__device__ inline uint32_t wait_word(const uint32_t* p, uint32_t* error) {
  uint32_t v, it = 0u;
  while ((v = ld_agent_u32(p)) == 0u) {
    __builtin_amdgcn_s_sleep(1);
    if (++it > kSpinLimit) {
      flag_error(error, kErrWait);
      return 0u;
    }
  }
  return v - 1u;
}

// A float as a handoff word: bits + 1, never 0 (the all-ones NaN pattern,
// which arithmetic never produces, is stored as the canonical NaN).
__device__ inline uint32_t to_word(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (u == 0xFFFFFFFFu ? 0x7FC00000u : u) + 1u;
}

// Pages whose scores and page ids are staged in LDS (16 per thread); longer
// rows are read straight from global memory.
constexpr uint32_t kStageMaxPages = 16u * kThreads;

struct TopkShared {
  alignas(16) uint32_t hist[3][kThreads];  // radix histograms, rotating over 3 buffers
  alignas(16) uint32_t key[kStageMaxPages];  // staged order keys, then the output
  int32_t id[kStageMaxPages];                // staged page ids
  uint32_t red[8];
  uint32_t s4[4];
};

struct RadixResult {
  uint32_t hmask;    // bits of (key - kmin) that decide the bucket (~0u << hi)
  uint32_t thr;      // the bucket of the k-th key: (key - kmin) & hmask == thr
  uint32_t kr;       // keys still to take from that bucket
  bool take_bucket;  // the bucket is taken whole (else: hi == 0, equal keys)
};

// Finds the bucket holding the kr-th largest free key (free_mask bit j: key[j]
// takes part) by a radix select over key - kmin, 8-bit digits from the top
// set bit of kmax - kmin down (one head's scores span a narrow range, so the
// first digit already spreads the keys); it stops as soon as the bucket of
// the kr-th key is taken whole.  One barrier per pass: the histogram is
// scanned by every wave, and buffers rotate over three, so the buffer cleared
// in pass i was last read in pass i-2, before the barrier of pass i-1.
// hist[0] must be zero on entry.
template <int KPT, typename Mask>
__device__ __forceinline__ RadixResult radix_select(const uint32_t (&rel)[KPT], Mask free_mask,
                                                    uint32_t range, uint32_t kr, TopkShared& sh) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = __lane_id();
  uint32_t prefix = 0u;
  int hi = range == 0u ? 0 : 32 - __builtin_clz(range);
  bool take_bucket = false;
  uint32_t buf = 0;
  while (hi > 0) {
    const int w = hi < 8 ? hi : 8;
    const int sft = hi - w;
    const uint32_t hmask = hi >= 32 ? 0u : ~0u << hi;
    // every key adds 1 to its bin if it takes part, else 0: no per-key
    // branch (keys that do not take part land on scattered bins)
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const bool part = ((free_mask >> j) & (Mask)1) && ((rel[j] ^ prefix) & hmask) == 0u;
      atomicAdd(&sh.hist[buf][(rel[j] >> sft) & ((1u << w) - 1u)], part ? 1u : 0u);
    }
    const uint32_t nxt = buf == 2u ? 0u : buf + 1u;
    sh.hist[nxt][tid] = 0u;
    __syncthreads();
    // lane L holds bins 255-4L .. 252-4L (descending)
    const uint4 h = *reinterpret_cast<const uint4*>(&sh.hist[buf][252u - 4u * lane]);
    const uint32_t s4 = (h.x + h.y) + (h.z + h.w);
    const uint32_t incl = wave_incl_scan(s4);
    const uint32_t excl = incl - s4;
    const bool hit = excl < kr && kr <= incl;  // exactly one lane
    const uint32_t c0 = excl + h.w, c1 = c0 + h.z, c2 = c1 + h.y;
    const uint32_t j = kr <= c0 ? 0u : kr <= c1 ? 1u : kr <= c2 ? 2u : 3u;
    const uint32_t above_l = j == 0u ? excl : j == 1u ? c0 : j == 2u ? c1 : c2;
    const uint32_t count_l = j == 0u ? h.w : j == 1u ? h.z : j == 2u ? h.y : h.x;
    const uint32_t src = (uint32_t)__builtin_ctzll(__builtin_amdgcn_ballot_w64(hit));
    const uint32_t jj = (uint32_t)__builtin_amdgcn_readlane((int)j, (int)src);
    const uint32_t above = (uint32_t)__builtin_amdgcn_readlane((int)above_l, (int)src);
    const uint32_t count = (uint32_t)__builtin_amdgcn_readlane((int)count_l, (int)src);
    prefix |= (255u - 4u * src - jj) << sft;
    kr -= above;
    hi = sft;
    buf = nxt;
    TL(kTlPass1);
    if (count == kr) {  // every key of the bucket is selected
      take_bucket = true;
      break;
    }
  }
  const uint32_t hmask = hi >= 32 ? 0u : ~0u << hi;
  return RadixResult{hmask, prefix & hmask, kr, take_bucket};
}

// Selects k of P pages from fp32 `scores` (filter_util.py:373-380): with
// `fixed`, pages 0 and P-1 always; the rest by descending score, ties to the
// lower page index.  Writes kv_ids[page] of the selected pages to out[] in
// ascending page order (agent-coherent stores).
//
// Thread t owns pages [t*kpt, t*kpt + kpt) as register keys, kpt <= KPT and
// P <= 256 * KPT.  With KPT <= 16 scores and ids are first copied to LDS
// with coalesced loads and the output is compacted in LDS and stored
// coalesced; with KPT = 64 (rows up to 16384 pages) keys are read and the
// output written per thread.
//
// SELF (one-launch layer): every decode workgroup of the kv head (of each
// query head of its group) runs this same selection on the same score words.
// The words are only read (a merging workgroup clears them), their
// wait starts with one sentinel word per scoring chunk, and the output stays
// in sh.key[0, k) for the caller (nothing is stored).
template <int KPT, bool SELF = false>
__device__ __forceinline__ void topk_block(const float* __restrict__ scores, uint32_t P, uint32_t k,
                                           bool fixed, const int32_t* __restrict__ kv_ids,
                                           int32_t* __restrict__ out, TopkShared& sh,
                                           uint32_t* hout, uint32_t hstride, uint32_t hcopies,
                                           uint32_t* hwords = nullptr, uint32_t* error = nullptr) {
  // page i of the output, also as id + 1 into the hcopies handoff rows
  auto put = [&](uint32_t i, int32_t id) {
    st_agent_i32(out + i, id);
    if (hout != nullptr)
      for (uint32_t c = 0; c < hcopies; ++c) st_agent_u32(hout + c * hstride + i, (uint32_t)id + 1u);
  };
  constexpr bool kStaged = KPT <= 16;
  static_assert(KPT % 4 == 0 && (KPT <= 16 || KPT == 64), "keys per thread");
  using Mask = typename std::conditional<(KPT > 32), uint64_t, uint32_t>::type;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = __lane_id();
  const uint32_t wave = tid / kWave;
  if (!SELF && hwords != nullptr && (k == 0u || k >= P)) {
    // the scores are not needed, but their handoff words must be consumed
    for (uint32_t i = tid; i < P; i += kThreads) {
      uint32_t it = 0u;
      for (; ld_agent_u32(hwords + i) == 0u && it < kSpinLimit; ++it) __builtin_amdgcn_s_sleep(1);
      // a word written after this gave up would be left set
      if (it >= kSpinLimit) flag_error(error, kErrWait);
      st_agent_u32(hwords + i, 0u);
    }
  }
  if (k == 0u) return;  // (quest_kernel convention with a budget of one page)
  if (k >= P) {  // everything selected
    for (uint32_t i = tid; i < P; i += kThreads) put(i, kv_ids[i]);
    return;
  }
  // kpt rounded up to 4 so staged keys are read as 16-byte LDS vectors
  const uint32_t kpt = kStaged ? (((P + kThreads - 1) / kThreads + 3u) & ~3u)
                               : (P + kThreads - 1) / kThreads;
  const uint32_t i0 = tid * kpt;
  const uint32_t nforced = fixed ? (P == 1u ? 1u : 2u) : 0u;
  auto is_free = [&](uint32_t i) { return !(fixed && (i == 0u || i == P - 1u)); };
  sh.hist[0][tid] = 0u;

  uint32_t key[KPT];
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
  if constexpr (kStaged) {
    // coalesced copy: all loads issued before any is used
    float sv[KPT];
    int32_t iv[KPT];
    if (hwords == nullptr) {
#pragma unroll
      for (int m = 0; m < KPT; ++m) {  // unconditional loads of clamped indices
        uint32_t i = tid + (uint32_t)m * kThreads;
        i = i < P ? i : P - 1u;
        sv[m] = ld_agent(scores + i);
        iv[m] = kv_ids[i];
      }
#ifdef AOAKV_TIMELINE
      // (noted once the loads have returned)
      if (__builtin_bit_cast(uint32_t, sv[KPT - 1]) != 0x7FBADBADu) TL(kTlRowLoaded);
#endif
    } else {
      // page ids first, then this thread's score words, polled until the
      // scoring items have written them, then cleared for the next launch
      // (only the thread owning a word clears it; clamped reads of another
      // thread's word are not used)
      uint32_t w[KPT];
#pragma unroll
      for (int m = 0; m < KPT; ++m) {
        uint32_t i = tid + (uint32_t)m * kThreads;
        i = i < P ? i : P - 1u;
        iv[m] = kv_ids[i];
      }
      if constexpr (SELF) {
        // first the head's last score word alone, so that the workgroups
        // waiting for a head poll one cache line each, not the whole row
        // (512 workgroups polling every word, or one word per scoring chunk,
        // cost 1.2 or 0.2 us per layer in memory traffic at config 2)
        if (wave == 0u) {
          const uint32_t* sw = hwords + (P - 1u);
          uint32_t it = 0u;
          for (; it < kSpinLimit; ++it) {
            if (__builtin_amdgcn_ballot_w64(ld_agent_u32(sw) == 0u) == 0u) break;
            __builtin_amdgcn_s_sleep(1);
          }
          if (it >= kSpinLimit && lane == 0u) flag_error(error, kErrWait);
        }
        __syncthreads();
        TL(kTlScoresSeen);
      }
      auto load_words = [&]() {
#pragma unroll
        for (int m = 0; m < KPT; ++m) {
          uint32_t i = tid + (uint32_t)m * kThreads;
          i = i < P ? i : P - 1u;
          w[m] = ld_agent_u32(hwords + i);
        }
      };
      auto missing = [&]() {
        bool z = false;
#pragma unroll
        for (int m = 0; m < KPT; ++m) z |= tid + (uint32_t)m * kThreads < P && w[m] == 0u;
        return z;
      };
      load_words();
      uint32_t it = 0u;
      for (; missing(); ++it) {
        if (it >= kSpinLimit) break;  // stand-in scores
        __builtin_amdgcn_s_sleep(1);
        load_words();
      }
      // a wait that gave up is flagged here, outside the poll loop (an atomic
      // inside it made this loop's code 0.4 us per layer slower): words
      // written after it are left set, and the next launch must not run on
      // them
      if (it >= kSpinLimit) flag_error(error, kErrWait);
      TL(kTlRowLoaded);
#pragma unroll
      for (int m = 0; m < KPT; ++m) {
        const uint32_t i = tid + (uint32_t)m * kThreads;
        if (!SELF && i < P) st_agent_u32(hwords + i, 0u);
        sv[m] = __builtin_bit_cast(float, w[m] - 1u);
      }
    }
    // no per-key branch: entries past P (inside the staging arrays, which
    // hold 256 * KPT) are written too and never read as valid keys
#pragma unroll
    for (int m = 0; m < KPT; ++m) {
      const uint32_t i = tid + (uint32_t)m * kThreads;
      const uint32_t kk = order_key(sv[m]);
      sh.key[i] = kk;
      sh.id[i] = iv[m];
      const bool use = i < P && is_free(i);
      kmin = use && kk < kmin ? kk : kmin;
      kmax = use && kk > kmax ? kk : kmax;
    }
  } else {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const uint32_t i = i0 + j;
      const bool valid = (uint32_t)j < kpt && i < P;
      key[j] = order_key(ld_agent(scores + (valid ? i : P - 1u)));
      if (valid && is_free(i)) {
        kmin = key[j] < kmin ? key[j] : kmin;
        kmax = key[j] > kmax ? key[j] : kmax;
      }
    }
  }
  kmin = wave_reduce_u32<false>(kmin);
  kmax = wave_reduce_u32<true>(kmax);
  if (lane == 0) {
    sh.red[wave] = kmin;
    sh.red[4 + wave] = kmax;
  }
  __syncthreads();
  TL(kTlStaged);
  kmin = sh.red[0];
  kmax = sh.red[4];
#pragma unroll
  for (int w4 = 1; w4 < 4; ++w4) {
    kmin = sh.red[w4] < kmin ? sh.red[w4] : kmin;
    kmax = sh.red[4 + w4] > kmax ? sh.red[4 + w4] : kmax;
  }
  if constexpr (kStaged) {
#pragma unroll
    for (int c = 0; c < KPT / 4; ++c) {
      const uint4 v = *reinterpret_cast<const uint4*>(&sh.key[i0 + 4u * c]);
      key[4 * c + 0] = v.x;
      key[4 * c + 1] = v.y;
      key[4 * c + 2] = v.z;
      key[4 * c + 3] = v.w;
    }
  }
  Mask free_mask = 0, valid_mask = 0;  // bit j: page i0+j exists / is not forced
  uint32_t rel[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const uint32_t i = i0 + j;
    rel[j] = key[j] - kmin;
    const bool v = (uint32_t)j < kpt && i < P;
    valid_mask |= (Mask)v << j;
    free_mask |= (Mask)(v && is_free(i)) << j;
  }
  // >= 1: k == 0 returned above, and with fixed forcing k >= 3 > nforced
  const RadixResult rr = radix_select<KPT, Mask>(rel, free_mask, kmax - kmin, k - nforced, sh);
  TL(kTlSelected);

  // selection classes at the final resolution:
  //   above:  forced, or (rel & hmask) > thr  -- selected
  //   bucket: (rel & hmask) == thr            -- rr.kr of them selected: all when
  //           take_bucket, else (equal keys) the lowest pages first
  Mask above_m = 0, eq_m = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const bool v = (valid_mask >> j) & 1u, f = (free_mask >> j) & 1u;
    const uint32_t r = rel[j] & rr.hmask;
    above_m |= (Mask)(v && (!f || r > rr.thr)) << j;
    eq_m |= (Mask)(v && f && r == rr.thr) << j;
  }
  // one scan of (pages above, bucket pages) packed in 16-bit halves gives the
  // output position: selected pages before mine = above before + min(bucket
  // pages before, kr)
  const uint32_t na = (uint32_t)__builtin_popcountll((uint64_t)above_m);
  const uint32_t ne = (uint32_t)__builtin_popcountll((uint64_t)eq_m);
  const uint32_t packed = na | (ne << 16);
  // this thread's page ids, read before the barrier below (after it, the id
  // array takes the discarded writes of the compaction)
  int32_t myid[kStaged ? KPT : 1];
  if constexpr (kStaged) {
#pragma unroll
    for (int c = 0; c < KPT / 4; ++c) {
      const int4 v = *reinterpret_cast<const int4*>(&sh.id[i0 + 4u * c]);
      myid[4 * c + 0] = v.x;
      myid[4 * c + 1] = v.y;
      myid[4 * c + 2] = v.z;
      myid[4 * c + 3] = v.w;
    }
  }
  const uint32_t incl = wave_incl_scan(packed);
  if (lane == kWave - 1) sh.s4[wave] = incl;
  __syncthreads();
  uint32_t before = incl - packed;
#pragma unroll
  for (uint32_t w4 = 0; w4 < 4; ++w4) before += w4 < wave ? sh.s4[w4] : 0u;
  const uint32_t eq_before = before >> 16;
  uint32_t pos = (before & 0xFFFFu) + (eq_before < rr.kr ? eq_before : rr.kr);
  uint32_t eq_rank = eq_before;
  if constexpr (kStaged) {
    // every key and id read from LDS finished before the barrier above, so
    // sh.key takes the compacted output and sh.id[tid] the discarded writes
    // (every key writes somewhere: no per-key branch)
    uint32_t* s_out = sh.key;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const bool eq = (eq_m >> j) & 1u;
      const bool take = ((above_m >> j) & 1u) || (eq && (rr.take_bucket || eq_rank < rr.kr));
      eq_rank += eq ? 1u : 0u;
      uint32_t* dst = take ? &s_out[pos] : reinterpret_cast<uint32_t*>(&sh.id[tid]);
      *dst = (uint32_t)myid[j];
      pos += take ? 1u : 0u;
    }
    __syncthreads();
    if (!SELF)
      for (uint32_t i = tid; i < k; i += kThreads) put(i, (int32_t)s_out[i]);
    TL(kTlOutput);
  } else {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      bool take = (above_m >> j) & 1u;
      if ((eq_m >> j) & 1u) take = rr.take_bucket || eq_rank++ < rr.kr;
      if (take) put(pos++, kv_ids[i0 + j]);
    }
  }
}

// top-k of a row of P <= kStageMaxPages pages with the fewest keys per thread
template <bool SELF = false>
__device__ __forceinline__ void topk_staged(const float* __restrict__ scores, uint32_t P, uint32_t k,
                                            bool fixed, const int32_t* __restrict__ kv_ids,
                                            int32_t* __restrict__ out, TopkShared& sh,
                                            uint32_t* hout = nullptr, uint32_t hstride = 0u,
                                            uint32_t hcopies = 0u, uint32_t* hwords = nullptr,
                                            uint32_t* error = nullptr) {
  if (P <= 4u * kThreads)
    topk_block<4, SELF>(scores, P, k, fixed, kv_ids, out, sh, hout, hstride, hcopies, hwords,
                          error);
  else if (P <= 8u * kThreads)
    topk_block<8, SELF>(scores, P, k, fixed, kv_ids, out, sh, hout, hstride, hcopies, hwords,
                          error);
  else
    topk_block<16, SELF>(scores, P, k, fixed, kv_ids, out, sh, hout, hstride, hcopies, hwords,
                          error);
}

// Pages per head the fused estimate + top-k kernel selects from (16 keys per
// thread keep its register count at the scoring kernel's); longer sequences
// use the standalone top-k kernel.
constexpr uint32_t kFusedTopkMaxPages = kStageMaxPages;

// ======================================================================
// page scores (+ optional fused top-k)
// ======================================================================

// Grid (page chunks of 128 / GROUP, kv heads, batch); a wave scores 32 /
// GROUP consecutive pages, one or (GROUP = 1) two metadata pages (page_size
// 16), so its metadata page indices are one or two scalar loads.
struct EstShared {
  float sc[kEstPagesPerBlock];
  uint32_t last;
};
struct EstTopkShared {
  EstShared e;
  TopkShared tk;
};

// Pages of sequence b the scoring covers: never past a score row or the
// max_pages the grid covers, and within the fused top-k's limit when fused.
// *clamped (if given) tells whether the page table held more.
__device__ inline uint32_t est_pages(const EstimateArgs& a, uint32_t b, uint32_t* pbeg_out,
                                     bool* clamped = nullptr) {
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P0 = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  uint32_t P = P0;
  // a score row holds a score per page, or per page but the last with the
  // quest_kernel convention (the last page is not scored)
  const uint32_t rowcap = a.score_stride + ((a.flags & kFlagQuestKernel) ? 1u : 0u);
  if (P > rowcap) P = rowcap;
  if (P > a.max_pages) P = a.max_pages;
  if (P > kFusedTopkMaxPages && a.sel != nullptr) P = kFusedTopkMaxPages;
  *pbeg_out = pbeg;
  if (clamped != nullptr) *clamped = P != P0;
  return P;
}

// Scores pages [n*chunk, n*chunk + n) of (sequence b, kv head h), n =
// kPPB, and stores them (agent-coherent).  With HPI = 2 (NHD layout, GROUP
// 1) the item covers kv heads h and h + 1 and kPPB pages of each: a step's
// four rows read pages p and p + 1 of both heads, so each pair of rows reads
// one 512-byte run (the two heads' adjacent 256-byte entries) instead of
// two 256-byte pieces 8 KB apart.  Returns false, uniformly, when the chunk
// holds no page.  A sequence whose page table exceeds what the call covers
// sets kErrTruncated (once, from its first chunk).
template <int GROUP, uint32_t kPPB = est_block_pages<GROUP>(), int HPI = 1>
__device__ __forceinline__ bool score_item(const EstimateArgs& a, uint32_t b, uint32_t h,
                                           uint32_t chunk, EstShared& sm) {
  static_assert(HPI == 1 || (HPI == 2 && GROUP == 1 && kPPB == 64u), "head pairs: GROUP 1");
  float* s_sc = sm.sc;
  const uint32_t lane = __lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t row = lane / kLanesPerRow;
  const uint32_t l16 = lane % kLanesPerRow;
  uint32_t pbeg;
  bool clamped;
  const uint32_t P = est_pages(a, b, &pbeg, &clamped);
  constexpr uint32_t kPPW = kPPB / 4u;  // pages per wave: 32, 16, 8 or 4
  static_assert(kPPW % 4u == 0u && kPageSize % kPPW == 0u || kPPW == 2u * kPageSize,
                "a wave's pages lie in one or two metadata pages");
  // step s, row r: page page0 + kPS * s + (r >> (HPI - 1)) of head h + (r & (HPI - 1))
  constexpr uint32_t kPS = 4u / (uint32_t)HPI;                   // pages per step
  const uint32_t rpage = row >> (HPI - 1), hrow = h + (row & (uint32_t)(HPI - 1));
  if (chunk * kPPB >= P) return false;  // uniform per block
  if (clamped && chunk == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  const uint32_t mbeg = (uint32_t)a.meta_indptr[b];
  const uint32_t d0 = l16 * kVec;
  const bool value_aware = (a.flags & kFlagValueAware) != 0u;

  // Every load below is unconditional, with an address that always lies in
  // the sequence's pages: a page past P reads a page of this block (its
  // score is never stored).  A load under a lane-dependent condition would
  // make the compiler wait for it before issuing the next one.  Issue order:
  // the page id for the value statistic, the metadata page ids, q, the 16
  // metadata vectors, then the value statistic (used only after scoring).
  const uint32_t pblk = chunk * kPPB;  // < P
  const uint32_t page0 = pblk + wave * kPPW;
  // lane j (< 32) holds the value statistic of step j / 4, row j % 4
  uint32_t pj = page0 + (lane % (kPPW * HPI)) / HPI;
  pj = pj < P ? pj : P - 1u;
  const uint32_t hj = h + (lane % (uint32_t)HPI);
  const uint32_t phys_j = (uint32_t)a.kv_indices[pbeg + pj];
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order written here
  const uint32_t pl0 = page0 < P ? page0 : pblk;  // a live page of the wave's first half
  const uint32_t pl1 = pl0 + kPageSize < P ? pl0 + kPageSize : pl0;
  const uint32_t mp0 = (uint32_t)a.meta_indices[mbeg + pl0 / kPageSize];
  const uint32_t mp1 =
      kPPW > kPageSize ? (uint32_t)a.meta_indices[mbeg + pl1 / kPageSize] : mp0;

  // Per dim, the larger of q*Kmax and q*Kmin is q*Kmax where q >= 0 and
  // q*Kmin where q < 0 (Kmax >= Kmin; fp16 products are exact in fp32).  So
  // each pair of dims is one byte permute that picks Kmax or Kmin by the
  // sign of q (a lane-constant selector) and one v_dot2_f32_f16.  Sums start
  // at +0, so a page whose terms are all zero scores +0 as with fmaxf.
  half2v q2[GROUP][kVec / 2];
  uint32_t psel[GROUP][kVec / 2];  // v_perm_b32 selectors: src0 = Kmax, src1 = Kmin
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    const H8 qq = ld16(a.q + ((size_t)b * a.Hq + hrow * GROUP + g) * kHeadDim + d0);
#pragma unroll
    for (int m = 0; m < kVec / 2; ++m) {
      q2[g][m] = half_pair(qq, m);
      const bool lo = !((float)qq.v[2 * m] < 0.f), hi = !((float)qq.v[2 * m + 1] < 0.f);
      psel[g][m] = (lo ? 0x0504u : 0x0100u) | (hi ? 0x07060000u : 0x03020000u);
    }
  }

  constexpr int kSteps = (int)(kPPW / kPS);
  H8 kmx[kSteps], kmn[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    // page page0 + kPS * s + rpage: its metadata page and slot
    const uint32_t mp = (uint32_t)s * kPS < kPageSize ? mp0 : mp1;
    const size_t off =
        elem_off(a.g, mp, 0, hrow, (page0 + (uint32_t)s * kPS + rpage) % kPageSize) + d0;
    // each metadata vector is read by one item, once: non-temporal loads
    // (config 2: 21.33 -> 21.03 us per layer; GQA 32 / 8 over 32 rotated
    // layers: 15.37 -> 15.08.  Over 8 rotated layers, whose 134 MB stay in
    // the memory-side cache, plain loads were faster: 14.37 against 14.68)
    kmx[s] = ld16_nt(a.meta + off);
    kmn[s] = ld16_nt(a.meta + off + a.g.kv);
  }
  __builtin_amdgcn_sched_barrier(0);
  // without the value term v_log_norm may be null: read q instead (unused)
  const f16 lvn_raw = *(value_aware ? a.v_log_norm + (size_t)phys_j * a.Hkv + hj : a.q);

  float sc[kSteps];  // score of step s's page of this row (same in all lanes of the row)
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    float x[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < kVec / 2; ++m) {
        const uint32_t kx = __builtin_bit_cast(uint32_t, half_pair(kmx[s], m));
        const uint32_t kn = __builtin_bit_cast(uint32_t, half_pair(kmn[s], m));
        const half2v kb = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(kx, kn, psel[g][m]));
        acc = __builtin_amdgcn_fdot2(q2[g][m], kb, acc, false);
      }
      x[g] = row_sum16(acc);
    }
    if (value_aware) {
      // 2 * (bound / sqrt(d)), logsumexp over the group (+ 2 * log-norm below)
      float m = -INFINITY;
#pragma unroll
      for (int g = 0; g < GROUP; ++g) {
        x[g] = 2.0f * (x[g] / kSqrtHeadDim);
        m = fmaxf(m, x[g]);
      }
      float lse = x[0];
      if (GROUP > 1) {
        float se = 0.f;
#pragma unroll
        for (int g = 0; g < GROUP; ++g) se = se + expf(x[g] - m);
        lse = logf(se) + m;
      }
      sc[s] = lse;
    } else {
      float t = x[0];
#pragma unroll
      for (int g = 1; g < GROUP; ++g) t = t + x[g];
      sc[s] = t;
    }
  }
  const float lvn_lane = (float)lvn_raw;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    float score = sc[s];
    if (value_aware) score = score + 2.0f * __shfl(lvn_lane, s * 4 + (int)row);
    // s_sc: [HPI heads][kPPB pages]
    if (l16 == 0u)
      s_sc[(row & (uint32_t)(HPI - 1)) * kPPB + wave * kPPW + (uint32_t)s * kPS + rpage] = score;
  }
  __syncthreads();
  {
    constexpr uint32_t kNsc = kPPB * HPI;  // scores of the item (<= 128)
    const uint32_t j = threadIdx.x % kNsc;
    const uint32_t hh = j / kPPB;  // < HPI
    const uint32_t p = chunk * kPPB + j % kPPB;
    const uint32_t nstore = (a.flags & kFlagQuestKernel) ? P - 1u : P;
    const size_t bh = (size_t)b * a.Hkv + h + hh;
    if (threadIdx.x < kNsc && p < nstore) st_agent(a.scores + bh * a.score_stride + p, s_sc[j]);
    // the handoff words: copy c of the row by threads [c * kNsc, (c + 1) * kNsc)
    // (hscore_copies * kNsc <= 128: a copy per decode block of the group)
    if (a.hscore != nullptr && threadIdx.x < kNsc * a.hscore_copies && p < nstore) {
      const uint32_t c = threadIdx.x / kNsc;
      st_agent_u32(a.hscore + (bh * a.hscore_copies + c) * a.hscore_stride + p, to_word(s_sc[j]));
    }
  }

  return true;
}

// The shape of one sequence's top-k: candidate pages, how many to select,
// and whether the decode items will read the handoff rows.  Computed before
// the wait for the scores, so its page-table loads are off the critical path.
struct SelPlan {
  uint32_t P, pbeg, k;
  bool handoff;
};

__device__ __forceinline__ SelPlan plan_select(const EstimateArgs& a, uint32_t b) {
  SelPlan p;
  const uint32_t lpl = (uint32_t)a.kv_last_page_len[b];
  const uint32_t budget = a.token_budgets ? (uint32_t)a.token_budgets[b] : a.token_budget;
  p.P = est_pages(a, b, &p.pbeg);
  p.k = p.P == 0u ? 0u
                  : num_selected_pages((p.P - 1u) * kPageSize + lpl, budget, kPageSize, p.P,
                                       a.flags);
  if ((a.flags & kFlagQuestKernel) && p.P != 0u) {
    // the last page is attended without selection: k - 1 of the others
    p.P -= 1u;
    p.k -= 1u;
  }
  if (p.k > a.sel_stride) p.k = a.sel_stride;  // never write past a selection row
  // no handoff entries for a sequence the decode items skip (malformed
  // last-page length): nothing would read and clear them
  p.handoff = a.hsel != nullptr && lpl >= 1u && lpl <= (uint32_t)kPageSize;
  return p;
}

// Top-k of (sequence b, kv head h) from its stored scores, every chunk
// written, as planned by plan_select.
template <int GROUP>
__device__ __forceinline__ void select_item(const EstimateArgs& a, uint32_t b, uint32_t h,
                                            const SelPlan& pl, TopkShared& tk) {
  const uint32_t P = pl.P, k = pl.k, pbeg = pl.pbeg;
  const bool handoff = pl.handoff;
  // one handoff row per decode item of the kv head's group: GROUP / gi copies,
  // rows b * Hq + h * GROUP + c * gi (each item clears the row it reads)
  const uint32_t gi = a.hsel_gi > 1u ? a.hsel_gi : 1u;
  uint32_t* hout = handoff ? a.hsel + ((size_t)b * a.Hq + h * GROUP) * a.hsel_stride : nullptr;
  uint32_t* hwords =
      a.hscore ? a.hscore + ((size_t)b * a.Hkv + h) * a.hscore_copies * a.hscore_stride : nullptr;
  topk_staged(a.scores + ((size_t)b * a.Hkv + h) * a.score_stride, P, k,
              (a.flags & kFlagFixed) != 0u, a.kv_indices + pbeg,
              a.sel + ((size_t)b * a.Hkv + h) * a.sel_stride, tk, hout, a.hsel_stride * gi,
              GROUP / gi, hwords, a.error);
}

// Scores one chunk; with a.sel set, the last block of the head to finish
// also selects its pages (arrival counter per head).
template <int GROUP, bool FUSED>
__device__ __forceinline__ void estimate_item(const EstimateArgs& a, uint32_t b, uint32_t h,
                                              uint32_t chunk, EstShared& sm, TopkShared* tk) {
  // the fused top-k's shape, loaded up front (off the handoff path)
  SelPlan plan{};
  if (a.sel != nullptr) plan = plan_select(a, b);
  constexpr uint32_t kPPB = est_kernel_block_pages<GROUP, FUSED>();
  if (!score_item<GROUP, kPPB>(a, b, h, chunk, sm)) return;
  if (a.sel == nullptr) return;
  uint32_t pbeg;
  const uint32_t nch = (est_pages(a, b, &pbeg) + kPPB - 1u) / kPPB;
  if (!arrive_last(&a.counters[(b * a.Hkv + h) * kCounterStride], nch, &sm.last)) return;
  select_item<GROUP>(a, b, h, plan, *tk);
}

template <int GROUP, bool FUSED>
__global__ __launch_bounds__(kThreads) void estimate_kernel(EstimateArgs a) {
  if constexpr (FUSED) {
    __shared__ EstTopkShared sm;
    estimate_item<GROUP, true>(a, blockIdx.z, blockIdx.y, blockIdx.x, sm.e, &sm.tk);
  } else {
    __shared__ EstShared sm;
    a.sel = nullptr;
    estimate_item<GROUP, false>(a, blockIdx.z, blockIdx.y, blockIdx.x, sm, nullptr);
  }
}

#ifdef AOAKV_TIMELINE
__device__ __forceinline__ void topk_body(const TopkArgs& a);

__global__ __launch_bounds__(kThreads) void topk_kernel(TopkArgs a) {
  TL_BEGIN();
  TL(kTlStart);
  topk_body(a);
  TL_FLUSH();
}

__device__ __forceinline__ void topk_body(const TopkArgs& a)
#else
__global__ __launch_bounds__(kThreads) void topk_kernel(TopkArgs a)
#endif
{
  __shared__ TopkShared sh;
  const uint32_t h = blockIdx.x, b = blockIdx.y;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  uint32_t P = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  if (P == 0u) return;
  const bool quest = (a.flags & kFlagQuestKernel) != 0u;
  const uint32_t rowcap = a.score_stride + (quest ? 1u : 0u);  // see est_pages
  // candidates are the pages the score row holds (as the reference's top-k
  // over an [H, n] row); a longer page table is flagged where there is a
  // workspace (the entry point checks score_stride against kTopkMaxPages)
  const uint32_t P0 = P;
  if (P > rowcap) P = rowcap;
  if (P > kTopkMaxPages) P = kTopkMaxPages;
  if (P != P0 && h == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  const uint32_t L = (P - 1u) * a.S + (uint32_t)a.kv_last_page_len[b];
  const uint32_t budget = a.token_budgets ? (uint32_t)a.token_budgets[b] : a.token_budget;
  uint32_t k = num_selected_pages(L, budget, a.S, P, a.flags);
  if (quest) {  // the last page is attended without selection
    P -= 1u;
    k -= 1u;
  }
  if (k > a.sel_stride) k = a.sel_stride;
  const bool fixed = (a.flags & kFlagFixed) != 0u;
  const float* row = a.scores + ((size_t)b * a.Hkv + h) * a.score_stride;
  int32_t* out = a.sel + ((size_t)b * a.Hkv + h) * a.sel_stride;
  if (P <= kStageMaxPages)
    topk_staged(row, P, k, fixed, a.kv_indices + pbeg, out, sh);
  else
    topk_block<kTopkMaxPages / kThreads>(row, P, k, fixed, a.kv_indices + pbeg, out, sh, nullptr,
                                          0u, 0u);
}

// ======================================================================
// sparse decode attention, split-K over pages with a fused merge
// ======================================================================

// out[u] = v of lane u of this lane's 16-lane row, u < 8 (DPP row_newbcast)
__device__ __forceinline__ void row_bcast8(float v, float (&out)[8]) {
  const int x = __builtin_bit_cast(int, v);
  out[0] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x150, 0xF, 0xF, false));
  out[1] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x151, 0xF, 0xF, false));
  out[2] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x152, 0xF, 0xF, false));
  out[3] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x153, 0xF, 0xF, false));
  out[4] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x154, 0xF, 0xF, false));
  out[5] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x155, 0xF, 0xF, false));
  out[6] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x156, 0xF, 0xF, false));
  out[7] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x157, 0xF, 0xF, false));
}

// out[i] = lane 2i of v's DPP row, in every lane of the row (row_newbcast)
__device__ __forceinline__ void row_bcast_even8(float v, float (&out)[8]) {
  const int x = __builtin_bit_cast(int, v);
  out[0] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x150, 0xF, 0xF, false));
  out[1] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x152, 0xF, 0xF, false));
  out[2] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x154, 0xF, 0xF, false));
  out[3] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x156, 0xF, 0xF, false));
  out[4] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x158, 0xF, 0xF, false));
  out[5] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x15A, 0xF, 0xF, false));
  out[6] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x15C, 0xF, 0xF, false));
  out[7] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x15E, 0xF, 0xF, false));
}

// G query heads per workgroup (the kv head's group): per wave and head the
// softmax statistics and output, then the workgroup's combined partials.
template <int G>
struct DecShared {
  float o[4][G][kHeadDim];
  float ml[4][G][2];
  float own[G][kHeadDim + 2];  // the merging block's own partials (one-launch layer)
  uint32_t sel[kDecPagesPerBlock];
  uint32_t last;
};

// Attends pages [8*chunk, 8*chunk + 8) of the selection of (sequence b, kv
// head hq0 / group) for the G query heads hq0 .. hq0 + G - 1 of that kv
// head's group: the K/V tiles are loaded once and stay in registers while each
// head's logits, softmax and weighted sum run over them.  G = 1 gives each
// query head its own workgroups (the default: the query heads of a group land
// on one XCD, 16 or a multiple of 8 workgroup indices apart, so they share the
// tiles through its L2 while running in parallel); G = group is the
// reference's decode block, one threadIdx.y per query head of the group
// (decode_attn.cuh:497-500).  Then the chunks are merged per query head.
//   HANDOFF = false (two launches): the selection comes from the previous
//     launch; chunks hand their partials (o, m, l) to the last block to
//     arrive at a per-(sequence, kv head) counter.
//   HANDOFF = true (one launch): the selection is read from the handoff rows
//     the kv head's top-k writes in this launch, each entry polled until
//     written; partials go to handoff words and the last chunk polls them
//     and merges.  Every block only waits on blocks with smaller indices,
//     which were dispatched before it.
//   SELF (one launch): instead of polling a selection, the workgroup runs the
//     kv head's top-k itself from the score words (every chunk of the head
//     computes the same selection) and keeps its entries; the merging chunk
//     clears the score words at the end.  With G < group each block of G
//     query heads reads a copy of its own (hscore_copies = group / G rows
//     per kv head), so its merging chunk clears that copy without waiting
//     for the group's other heads.
// QUEST (quest_kernel convention): the selection rows hold the pages chosen
// besides the last page, which is always attended as the final entry
// (quest/utils/__init__.py:237, approx_attn.cu:68-151).
// One launch: err0 is the error word as read at the workgroup's start and
// s_err an LDS word for it; with kErrWait set no handoff word is touched and
// the group's outputs are NaN (written by its chunk 0).
template <bool HANDOFF, bool QUEST, bool SELF = false, int G = 1, bool STREAM = false>
__device__ __forceinline__ void decode_item(const DecodeArgs& a, uint32_t b, uint32_t hq0,
                                            uint32_t chunk, DecShared<G>& sm,
                                            const EstimateArgs* ea = nullptr,
                                            TopkShared* tk = nullptr, uint32_t* s_err = nullptr,
                                            uint32_t err0 = 0u) {
  // SELF without HANDOFF (the two-launch decode): the scores are complete
  // (written by the previous launch), read as floats, nothing to wait for
  // or clear
  const uint32_t lane = __lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t row = lane / kLanesPerRow;
  const uint32_t l16 = lane % kLanesPerRow;
  const uint32_t S = kPageSize;
  const uint32_t d0 = l16 * kVec;
  const uint32_t group = a.Hq / a.Hkv;
  const uint32_t hkv = hq0 / group;
  const size_t bh0 = (size_t)b * a.Hq + hq0;  // the item's first query head
  const uint32_t idx0 = chunk * kDecPagesPerBlock + wave * kDecPagesPerWave;
  const uint32_t* sel_row =
      a.sel ? reinterpret_cast<const uint32_t*>(a.sel) + ((size_t)b * a.Hkv + hkv) * a.sel_stride
            : nullptr;
  // Loads are unconditional with clamped addresses and masked afterwards (a
  // load under a lane- or page-dependent condition makes the compiler wait
  // for it before issuing the next).  The page-table words, the selection
  // entries and q need no earlier load, so they are all issued first.
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P_table = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  // a page table longer than the call was sized for is cut where the
  // scoring cuts it (est_pages), so the selection's size and the decode's
  // agree; flagged once per (sequence, kv head)
  const uint32_t P = P_table < a.max_pages ? P_table : a.max_pages;
  const uint32_t lpl = (uint32_t)a.kv_last_page_len[b];
  const int32_t tbv = *(a.token_budgets ? a.token_budgets + b : a.kv_indptr + b);
  const uint32_t budget = a.token_budgets ? (uint32_t)tbv : a.token_budget;
  const uint32_t ich = chunk * kDecPagesPerBlock;  // the chunk's first entry
  uint32_t selv[kDecPagesPerWave], sel_ch = 0u;
  if (!HANDOFF) {
    // dense decode reads its page ids from kv_indices below; its
    // "selection" loads read kv_indptr[0] (never used)
    const uint32_t* sel_src = sel_row ? sel_row : reinterpret_cast<const uint32_t*>(a.kv_indptr);
    const uint32_t sel_last = sel_row ? a.sel_stride - 1u : 0u;
    sel_ch = ld_agent_u32(sel_src + (ich < sel_last ? ich : sel_last));
#pragma unroll
    for (int s = 0; s < kDecPagesPerWave; ++s)
      selv[s] = ld_agent_u32(sel_src + (idx0 + s < sel_last ? idx0 + s : sel_last));
  }
  H8 qq[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qq[g] = ld16(a.q + (bh0 + g) * kHeadDim + d0);
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order written here
  // SELF: the head's top-k shape and its score words
  SelPlan pl{};
  uint32_t* words = nullptr;
  if constexpr (SELF) {
    pl = plan_select(*ea, b);
    // this block's copy of the kv head's score words
    if (HANDOFF)
      words = ea->hscore + (((size_t)b * ea->Hkv + hkv) * ea->hscore_copies +
                            (ea->hscore_copies > 1u ? (hq0 % group) / (uint32_t)G : 0u)) *
                               ea->hscore_stride;
  }
  // waits until the score words [0, pl.P) are written, then clears them
  auto consume_words = [&]() {
    for (uint32_t i = threadIdx.x; i < pl.P; i += kThreads) {
      uint32_t it = 0u;
      for (; ld_agent_u32(words + i) == 0u && it < kSpinLimit; ++it) __builtin_amdgcn_s_sleep(1);
      if (it >= kSpinLimit) flag_error(a.error, kErrWait);  // a late word would be left set
      st_agent_u32(words + i, 0u);
    }
  };
  if constexpr (HANDOFF) {
    if (threadIdx.x == 0u) *s_err = err0;
    __syncthreads();
    if ((*s_err & kErrWait) != 0u) {
      if (chunk == 0u)
        for (uint32_t i = threadIdx.x; i < (uint32_t)(G * kHeadDim); i += kThreads)
          a.o[bh0 * kHeadDim + i] = (f16)__builtin_nanf("");
      return;
    }
  }
  if (P != P_table && chunk == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  if (P == 0u || lpl == 0u || lpl > S) {  // malformed page table
    // the words were written all the same: consumed once per kv head
    if (SELF && HANDOFF && chunk == 0u) consume_words();  // (this block's copy)
    return;
  }
  // physical id of the sequence's last page (the one holding lpl tokens)
  uint32_t last_phys = 0u;
  if constexpr (QUEST) last_phys = (uint32_t)a.kv_indices[pbeg + P - 1u];
  uint32_t npages = P;
  if (a.sel != nullptr) {
    npages = num_selected_pages((P - 1u) * S + lpl, budget, S, P,
                                QUEST ? kFlagQuestKernel : 0u);
    const uint32_t row_cap = a.sel_stride + (QUEST ? 1u : 0u);
    if (npages > row_cap) npages = row_cap;
  }
  // the grid holds max_chunks blocks per head; never index partials past it
  const uint32_t cap =
      a.max_chunks < (uint32_t)kMergeMaxChunks ? a.max_chunks : (uint32_t)kMergeMaxChunks;
  if (npages > cap * kDecPagesPerBlock) {  // more pages than the call was sized for
    npages = cap * kDecPagesPerBlock;
    if (chunk == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  }
  const uint32_t nch = (npages + kDecPagesPerBlock - 1) / kDecPagesPerBlock;
  if (chunk >= nch) return;  // uniform per block
  // entries [0, nsel) come from the selection; with QUEST the entry after
  // them is the last page
  const uint32_t nsel = (QUEST && a.sel != nullptr) ? npages - 1u : npages;
  bool self_topk = false;  // SELF: the entries came from this workgroup's top-k
  if constexpr (SELF) {
    // the head's selection, computed here: entries [0, nout), in page order
    const EstimateArgs& e = *ea;
    const int32_t* ids = e.kv_indices + pl.pbeg;
    self_topk = pl.k != 0u && pl.k < pl.P;
    if (self_topk)
      topk_staged<true>(HANDOFF ? nullptr : e.scores + ((size_t)b * e.Hkv + hkv) * e.score_stride,
                        pl.P, pl.k, (e.flags & kFlagFixed) != 0u, ids, nullptr, *tk, nullptr, 0u,
                        0u, words, a.error);
    const uint32_t nout = self_topk ? pl.k : (pl.k == 0u ? 0u : pl.P);
    // entry i (page 0 past the selection; an entry the top-k did not yield
    // means the shapes disagree: flagged like a wait that gave up)
    auto entry = [&](uint32_t i) -> uint32_t {
      if (i >= nsel) return 0u;
      if (i >= nout) {
        flag_error(a.error, kErrWait);
        return 0u;
      }
      return self_topk ? tk->key[i] : (uint32_t)ids[i];
    };
    sel_ch = entry(ich);
    TL(kTlSelInHand);
#pragma unroll
    for (int s = 0; s < kDecPagesPerWave; ++s) selv[s] = entry(idx0 + s);
    // this chunk's entries of the selection output (the last chunk also
    // writes any the decode does not cover)
    int32_t* sel_out = e.sel + ((size_t)b * e.Hkv + hkv) * e.sel_stride;
    const uint32_t o_end = chunk == nch - 1u ? nout : (ich + kDecPagesPerBlock < nout ? ich + kDecPagesPerBlock : nout);
    for (uint32_t i = ich + threadIdx.x; i < o_end; i += kThreads)
      sel_out[i] = (int32_t)(self_topk ? tk->key[i] : (uint32_t)ids[i]);
  } else if (HANDOFF) {
    // this chunk's entries of the kv head's selection, each polled until the
    // top-k of this launch has written it, then cleared for the next launch
    uint32_t* hrow = a.hsel + bh0 * a.hsel_stride;  // this item's copy
    const uint32_t e = ich + threadIdx.x;
    if (threadIdx.x < (uint32_t)kDecPagesPerBlock)
      sm.sel[threadIdx.x] = e < nsel ? wait_word(hrow + e, a.error) : 0u;
    __syncthreads();
    if (threadIdx.x < (uint32_t)kDecPagesPerBlock && e < nsel) st_agent_u32(hrow + e, 0u);
    sel_ch = sm.sel[0];
    TL(kTlSelInHand);
#pragma unroll
    for (int s = 0; s < kDecPagesPerWave; ++s) selv[s] = sm.sel[wave * kDecPagesPerWave + s];
  }

  // ---- K/V loads of this wave's pages; an entry past the selection reads
  // the chunk's first selected page instead (masked below)
  uint32_t phys[kDecPagesPerWave];
  bool live[kDecPagesPerWave];
#pragma unroll
  for (int s = 0; s < kDecPagesPerWave; ++s) {
    live[s] = idx0 + s < npages;
    if (a.sel != nullptr) {
      phys[s] = live[s] ? selv[s] : sel_ch;
      if (QUEST && idx0 + s >= nsel) phys[s] = last_phys;
    } else {
      const uint32_t i = live[s] ? idx0 + s : ich;
      phys[s] = (uint32_t)a.kv_indices[pbeg + i];
    }
  }
  // STREAM (no GQA: each selected page's K/V is read by this item alone):
  // non-temporal loads, config 2 21.33 -> 20.88 us per layer.  The query
  // heads of a GQA group read their kv head's pages through the L2, and
  // non-temporal loads there made the layer slower (32 / 8 over 32 rotated
  // layers, with streamed metadata: 15.08 -> 15.21 us)
  auto ldkv = [](const f16* p) { return STREAM ? ld16_nt(p) : ld16(p); };
  H8 kk[kDecPagesPerWave][4], vv[kDecPagesPerWave][4];
#pragma unroll
  for (int s = 0; s < kDecPagesPerWave; ++s) {
    const size_t kbase = elem_off(a.g, phys[s], 0, hkv, 0) + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) kk[s][i] = ldkv(a.kv + kbase + (size_t)(i * 4 + row) * a.g.tok);
  }
#pragma unroll
  for (int s = 0; s < kDecPagesPerWave; ++s) {
    const size_t vbase = elem_off(a.g, phys[s], 1, hkv, 0) + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) vv[s][i] = ldkv(a.kv + vbase + (size_t)(i * 4 + row) * a.g.tok);
  }
  __builtin_amdgcn_sched_barrier(0);
  // tokens per page: the sequence's last page holds lpl of them
  if constexpr (!QUEST) last_phys = (uint32_t)a.kv_indices[pbeg + P - 1u];
  uint32_t ntok[kDecPagesPerWave];
#pragma unroll
  for (int s = 0; s < kDecPagesPerWave; ++s)
    ntok[s] = live[s] ? (phys[s] == last_phys ? lpl : S) : 0u;
  bool v_zeroed = false;  // the V of slots past a page's tokens, zeroed once

  constexpr int kTok = kDecPagesPerWave * 4;
  static_assert(kTok == 8, "one rounding lane per token of a row");
  const uint32_t um = l16 % (uint32_t)kTok;  // this lane's token
#pragma unroll
  for (int g = 0; g < G; ++g) {
    // q as four fp16 pairs: each logit term pair is one v_dot2_f32_f16
    // (exact fp16 products, fp32 sum)
    half2v q2[kVec / 2];
#pragma unroll
    for (int m = 0; m < kVec / 2; ++m) q2[m] = half_pair(qq[g], m);
    // ---- logits: fp16(q.k), then fp16(. / sqrt(d))  (quest_attention.py:265-268).
    // The 16 lanes of a row hold the same 8 dot sums (tokens i*4 + row of the
    // wave's two pages, u = 4s + i); lane l16 % 8 rounds and exponentiates
    // token u = l16 % 8 only, and the row takes each token's value from its
    // lane with DPP row_newbcast (the same arithmetic per token, once).
    float raw[kTok];
#pragma unroll
    for (int s = 0; s < kDecPagesPerWave; ++s) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < kVec / 2; ++m)
          acc = __builtin_amdgcn_fdot2(q2[m], half_pair(kk[s][i], m), acc, false);
        raw[s * 4 + i] = row_sum16(acc);
      }
    }
    float pick = raw[0];
#pragma unroll
    for (int u = 1; u < kTok; ++u) pick = um == (uint32_t)u ? raw[u] : pick;
    float xm = (float)r16(div_sqrt_head_dim_f16((float)r16(pick)));
    xm = (um % 4u) * 4u + row < (um < 4u ? ntok[0] : ntok[1]) ? xm : -INFINITY;
    float x[kTok];
    row_bcast8(xm, x);
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < kTok; ++u) mloc = fmaxf(mloc, x[u]);
    const float m = cross_row_max(mloc);
    float lsum = 0.f;
    float o[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j) o[j] = 0.f;
    if (m != -INFINITY) {
      // slots past a page's token count (the sequence's last page) hold
      // whatever the cache held: their probability is exactly 0, but 0 * NaN
      // is NaN, so their V is zeroed.  A wave-uniform branch (every lane holds
      // the same two pages), taken for the last page and unused entries only,
      // and placed where the V loads are waited for anyway: a write to vv
      // right after its loads would make the compiler wait for them there.
      if (!v_zeroed && (ntok[0] < S || ntok[1] < S)) {
#pragma unroll
        for (int s = 0; s < kDecPagesPerWave; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if ((uint32_t)(i * 4) + row >= ntok[s]) vv[s][i] = H8{};
        v_zeroed = true;
      }
      float pv[kTok];
      row_bcast8(__expf(xm - m), pv);
#pragma unroll
      for (int u = 0; u < kTok; ++u) {
        const float p = pv[u];
        lsum = lsum + p;
        // one mixed-precision FMA per dim (fp16 V converted in the FMA)
#pragma unroll
        for (int j = 0; j < kVec; ++j) o[j] = __builtin_fmaf(p, (float)vv[u / 4][u % 4].v[j], o[j]);
      }
    }
    lsum = cross_row_sum(lsum);
#pragma unroll
    for (int j = 0; j < kVec; ++j) o[j] = cross_row_sum(o[j]);
    // this wave's (o, m, l) of head g
    if (row == 0u) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) sm.o[wave][g][d0 + j] = o[j];
      if (l16 == 0u) {
        sm.ml[wave][g][0] = m;
        sm.ml[wave][g][1] = lsum;
      }
    }
  }

  TL(kTlAttended);
  // ---- combine the 4 waves of the block in LDS, store the chunk's (o, m, l)
  // per query head
  __syncthreads();
  for (uint32_t idx = threadIdx.x; idx < (uint32_t)G * (kHeadDim + 2u); idx += kThreads) {
    const uint32_t g = G == 1 ? 0u : idx / (kHeadDim + 2u);
    const uint32_t d = G == 1 ? idx : idx % (kHeadDim + 2u);
    const float M = fmaxf(fmaxf(sm.ml[0][g][0], sm.ml[1][g][0]), fmaxf(sm.ml[2][g][0], sm.ml[3][g][0]));
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = sm.ml[w][g][0] == -INFINITY ? 0.f : __expf(sm.ml[w][g][0] - M);
      const float val = d < (uint32_t)kHeadDim ? sm.o[w][g][d] : sm.ml[w][g][1];
      acc = acc + sc * val;
    }
    // slots 0..127: o; slot 128: m; slot 129: l
    const float val = d == (uint32_t)kHeadDim ? M : acc;
    const size_t part_off = ((bh0 + g) * a.max_chunks + chunk) * kPartialStride;
    // the one-launch merging block (the head's last chunk) keeps its own
    // partials in LDS: no store, no poll of them
    if (!HANDOFF) st_agent(a.partial + part_off + d, val);
    else if (chunk == nch - 1u) sm.own[g][d] = val;
    else st_agent_u32(a.hpart + part_off + d, to_word(val));
  }

  TL(kTlPartial);
  // ---- one block of this (sequence, kv head) merges the chunks of each of
  // its query heads
  if (HANDOFF) {
    if (chunk != nch - 1u) return;  // the head's last chunk
    __syncthreads();                // its own partials are in LDS
  } else {
    if (!arrive_last(&a.counters[bh0 * kCounterStride], nch, &sm.last)) return;
  }
  const uint32_t d = threadIdx.x % kHeadDim, half = threadIdx.x / kHeadDim;
  const uint32_t nm = nch - 1u;  // chunks merged from memory
  // chunks in groups of 16, the G heads' words of a group loaded together:
  // every load of a group is issued before any is used (one memory round
  // trip per group, handoff words re-polled until written); thread t sums dim
  // t%128 over the chunks of parity t/128, with the group max folded in online.
  // The last chunk (nch - 1) is folded in after the others: in the one-launch
  // layer it is the merging block's own partial, from LDS.
  float M[G], Lsum[G], acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    M[g] = -INFINITY;
    Lsum[g] = 0.f;
    acc[g] = 0.f;
  }
  for (uint32_t g0 = 0; g0 < nm; g0 += 16u) {
    const uint32_t ng = nm - g0 < 16u ? nm - g0 : 16u;
    // unconditional loads of clamped chunk indices, masked after.  Lane j
    // loads chunk j % 16's m and l words (the wave's four rows hold the same
    // 16 chunks), so the group max, the chunk weights and the weighted sum
    // of l are formed across the 16 lanes of a row, not by every thread for
    // every chunk (32 readlanes, 16 exponentials and 16 products each)
    const uint32_t mlc = lane % 16u;
    uint32_t mw[G], lw[G], ow[G][8];
    auto load_group = [&]() {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const size_t gb = ((bh0 + g) * a.max_chunks + g0) * kPartialStride;
        {
          const uint32_t cc = mlc < ng ? mlc : ng - 1u;
          const size_t at = gb + cc * kPartialStride + kHeadDim;
          mw[g] = HANDOFF ? ld_agent_u32(a.hpart + at)
                          : __builtin_bit_cast(uint32_t, ld_agent(a.partial + at));
          lw[g] = HANDOFF ? ld_agent_u32(a.hpart + at + 1u)
                          : __builtin_bit_cast(uint32_t, ld_agent(a.partial + at + 1u));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t c = half + 2u * i;
          const size_t at = gb + (c < ng ? c : ng - 1u) * kPartialStride + d;
          ow[g][i] = HANDOFF ? ld_agent_u32(a.hpart + at)
                             : __builtin_bit_cast(uint32_t, ld_agent(a.partial + at));
        }
      }
    };
    load_group();
    if (HANDOFF) {
      // re-poll (the whole wave) until every word of the group it uses is
      // written, then decode
      auto missing = [&]() {
        bool z = false;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          z |= mlc < ng && (mw[g] == 0u || lw[g] == 0u);
#pragma unroll
          for (int i = 0; i < 8; ++i) z |= half + 2u * i < ng && ow[g][i] == 0u;
        }
        return __builtin_amdgcn_ballot_w64(z) != 0u;
      };
      uint32_t it = 0u;
      while (missing()) {
        if (++it > kSpinLimit) {
          flag_error(a.error, kErrWait);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        load_group();
      }
      TL(kTlMergeLoaded);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        mw[g] -= 1u;
        lw[g] -= 1u;
#pragma unroll
        for (int i = 0; i < 8; ++i) ow[g][i] -= 1u;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m_c = mlc < ng ? __builtin_bit_cast(float, mw[g]) : -INFINITY;
      const float l_c = mlc < ng ? __builtin_bit_cast(float, lw[g]) : 0.f;
      float ov[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) ov[i] = half + 2u * i < ng ? __builtin_bit_cast(float, ow[g][i]) : 0.f;
      const float Mn = fmaxf(M[g], row_max16(m_c));
      const float keep = M[g] == -INFINITY ? 0.f : __expf(M[g] - Mn);
      const float w_c = m_c == -INFINITY ? 0.f : __expf(m_c - Mn);  // chunk mlc's weight
      Lsum[g] = Lsum[g] * keep + row_sum16(w_c * l_c);
      acc[g] = acc[g] * keep;
      // this thread's chunks half + 2i: lane 2i of w_h's row holds chunk
      // half + 2i's weight (half is wave-uniform), broadcast with DPP
      const float w_h = half != 0u ? dpp<kRowShl1>(w_c) : w_c;
      float wt[8];
      row_bcast_even8(w_h, wt);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g] = acc[g] + wt[i] * ov[i];
      M[g] = Mn;
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {  // the last chunk
    float lm, ll, lo;
    if (HANDOFF) {
      lm = sm.own[g][kHeadDim];
      ll = sm.own[g][kHeadDim + 1];
      lo = sm.own[g][d];
    } else {
      const size_t at = ((bh0 + g) * a.max_chunks + nm) * kPartialStride;
      lm = ld_agent(a.partial + at + kHeadDim);
      ll = ld_agent(a.partial + at + kHeadDim + 1);
      lo = ld_agent(a.partial + at + d);
    }
    const float Mn = fmaxf(M[g], lm);
    const float keep = M[g] == -INFINITY ? 0.f : __expf(M[g] - Mn);
    Lsum[g] = Lsum[g] * keep;
    acc[g] = acc[g] * keep;
    const float w = lm == -INFINITY ? 0.f : __expf(lm - Mn);
    Lsum[g] = Lsum[g] + w * ll;
    if (half == (nm & 1u)) acc[g] = acc[g] + w * lo;  // the half that sums its parity
    if (half == 1u) sm.o[0][g][d] = acc[g];
  }
  __syncthreads();
  if (half == 0u) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      a.o[(bh0 + g) * kHeadDim + d] = r16((acc[g] + sm.o[0][g][d]) / Lsum[g]);
  }
  TL(kTlOutput);
  // Every thread has read its words (barriers above): clear them -- o words
  // by their reader, m / l words by thread c.  Handoff words must be zero for
  // the next launch; the two-launch partials are cleared as well, so the
  // whole workspace is zero between calls whatever its layout: region
  // offsets depend on the call's selection size, and a later call with a
  // smaller one places its handoff words where these partials were.
  uint32_t* pwords = HANDOFF ? a.hpart : reinterpret_cast<uint32_t*>(a.partial);
#pragma unroll 1
  for (uint32_t g = 0; g < (uint32_t)G; ++g) {
    const size_t base = (bh0 + g) * a.max_chunks * kPartialStride;
    for (uint32_t g0 = 0; g0 < nch; g0 += 16u) {
      const size_t gb = base + (size_t)g0 * kPartialStride;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t c = g0 + half + 2u * i;
        if (c < nch) st_agent_u32(pwords + gb + (half + 2u * i) * kPartialStride + d, 0u);
      }
      const uint32_t c = g0 + threadIdx.x;
      if (threadIdx.x < 16u && c < nch) {
        st_agent_u32(pwords + gb + threadIdx.x * kPartialStride + kHeadDim, 0u);
        st_agent_u32(pwords + gb + threadIdx.x * kPartialStride + kHeadDim + 1, 0u);
      }
    }
  }
  if constexpr (SELF && HANDOFF) {
    // every chunk's partial arrived, and each chunk stored its partial after
    // its top-k had read this block's copy of the score words: clear it
    // (without a top-k no one waited for them, so wait first)
    if (self_topk) {
      for (uint32_t i = threadIdx.x; i < pl.P; i += kThreads) st_agent_u32(words + i, 0u);
    } else {
      consume_words();
    }
  }
}

// grid (chunks, query heads / G, sequences).  SELF: no selection rows; every
// item runs its kv head's top-k on the scores the previous launch wrote (e:
// the scoring call's arguments with sel, budgets and flags) and writes its
// chunk's entries of the selection.
template <bool QUEST, int G, bool SELF = false, bool STREAM = false>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeArgs a, EstimateArgs e) {
  TL_BEGIN();
  TL(kTlStart);
  if constexpr (SELF) {
    __shared__ union {
      TopkShared tk;
      DecShared<G> d;
    } sm;
    decode_item<false, QUEST, true, G, STREAM>(a, blockIdx.z, blockIdx.y * G, blockIdx.x, sm.d,
                                               &e, &sm.tk);
  } else {
    __shared__ DecShared<G> sm;
    decode_item<false, QUEST, false, G, STREAM>(a, blockIdx.z, blockIdx.y * G, blockIdx.x, sm);
  }
  TL_FLUSH();
}

// ======================================================================
// one launch per decode layer
// ======================================================================
//
// Workgroups, in index order:
//   [0, n_workers)            scoring workers: item i = n_workers*r + w in
//                             rounds r, items head by head, so the heads
//                             finish one after another and the later steps
//                             of early heads overlap the scoring of later
//                             ones; each scored item bumps its head's count
//   [.., + n_heads)           one top-k per (sequence, kv head): waits for
//                             the head's count, selects, writes the handoff
//                             selection
//   [.., + n_dec)             decode items, head by head: poll their
//                             selection entries; the head's last chunk
//                             polls the other chunks' partials and merges
// Workgroups are dispatched in index order, so every wait is on workgroups
// that have already started and that never wait on later ones; each wait is
// bounded by kSpinLimit regardless (then the error flag is set).  Counters
// and handoff words are cleared by their readers, so the workspace is zero
// again for the next launch.  No counter is shared by all workgroups
// (same-address device atomics serialize at ~12 ns each).
// SELF (la.self_select): the decode items select for themselves; a separate
// instantiation, so the other path keeps its own register budget.  GI: query
// heads per decode item (1, or the whole group).  HPI: kv heads per scoring
// item (2: NHD head pairs, score_item; the heads' scores go out as words).
#ifdef AOAKV_TIMELINE
// the profiling build wraps the kernel body to note its start and write the
// notes out when the workgroup ends, whichever way the body returns
template <int GROUP, bool QUEST, bool SELF, int GI, int HPI = 1>
__device__ __forceinline__ void layer_body(const LayerArgs& la);

template <int GROUP, bool QUEST, bool SELF, int GI, int HPI = 1>
__global__ __launch_bounds__(kThreads) void layer_kernel(LayerArgs la) {
  TL_BEGIN();
  layer_body<GROUP, QUEST, SELF, GI, HPI>(la);
  TL_FLUSH();
}

template <int GROUP, bool QUEST, bool SELF, int GI, int HPI>
__device__ __forceinline__ void layer_body(const LayerArgs& la)
#else
template <int GROUP, bool QUEST, bool SELF, int GI, int HPI = 1>
__global__ __launch_bounds__(kThreads) void layer_kernel(LayerArgs la)
#endif
{
  static_assert(GI == 1 || GI == GROUP, "a decode item serves one query head or the group");
  static_assert(HPI == 1 || GROUP == 1, "head-paired scoring items: GROUP 1");
  __shared__ union {
    EstTopkShared e;
    DecShared<GI> d;
  } sm;
  __shared__ uint32_t s_ok;
  // The error word as the launch found it: kErrWait there means an earlier
  // launch's wait gave up and may have left handoff words set, so no
  // workgroup that reads handoff words (top-k workgroups, decode items)
  // touches one; they check the word, passed through s_err, before their
  // first handoff access, and the output is NaN until the caller
  // re-initialises the workspace.  Scoring workers only write words, which a
  // refusing reader never consumes, so they do not read it.  A plain load:
  // the previous launch's flag is visible after the kernel boundary, and
  // the read is served by each XCD's L2 rather than by one memory word for
  // every workgroup (a coherent load of it in all 992 workgroups of config
  // 2 cost 0.67 us per layer).
  __shared__ uint32_t s_err;
  const uint32_t t = blockIdx.x;
  TL(kTlStart);
  if (t < la.n_workers) {
    // the first item's head bh0 starts bh0 * stagger in (see layer_stagger_ps)
    sleep_until(__builtin_amdgcn_s_memrealtime(), (uint64_t)(t / la.est_chunks) * la.stagger_ps);
    TL(kTlStaggerDone);
    int tl_item = 0;
    for (uint32_t i = t; i < la.n_est; i += la.n_workers) {
      // bh: (sequence, kv head) -- or head pair, HPI = 2
      const uint32_t bh = i / la.est_chunks, chunk = i % la.est_chunks;
      const uint32_t hu = la.e.Hkv / HPI;  // scoring units per sequence
      const uint32_t b = bh / hu, h = (bh % hu) * HPI;
      if (score_item<GROUP, est_block_pages<GROUP>() / HPI, HPI>(la.e, b, h, chunk, sm.e.e)) {
        TL(tl_item == 0 ? kTlScored0 : kTlScored1);
        ++tl_item;
        (void)tl_item;
        if (SELF || HPI == 2 || la.e.hscore != nullptr) {  // (SELF, HPI 2: score words only)
          // the scores went out as handoff words: only end this item's use
          // of LDS before the next item's
          __syncthreads();
        } else {
          // the scores are stored once the memory counter drains; the
          // barrier also ends this item's use of LDS before the next item's
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();
          if (threadIdx.x == 0)
            __hip_atomic_fetch_add(la.e.counters + bh * kCounterStride, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  } else if (!SELF && t < la.n_workers + la.n_heads) {  // (SELF: no top-k workgroups)
    const uint32_t err0 = *la.d.error;
    const uint32_t bh = t - la.n_workers;
    const uint32_t b = bh / la.e.Hkv, h = bh % la.e.Hkv;
    uint32_t pbeg;
    const uint32_t P = est_pages(la.e, b, &pbeg);
    if (P == 0u) return;
    const uint32_t nch = (P + est_block_pages<GROUP>() - 1u) / est_block_pages<GROUP>();
    const SelPlan plan = plan_select(la.e, b);
    if (threadIdx.x == 0u) s_err = err0;
    __syncthreads();
    if ((s_err & kErrWait) != 0u) return;
    if (la.e.hscore != nullptr) {  // the top-k polls the score words itself
      select_item<GROUP>(la.e, b, h, plan, sm.e.tk);
      return;
    }
    if (threadIdx.x == 0) {
      uint32_t it = 0u, ok = 1u;
      while (ld_agent_u32(la.e.counters + bh * kCounterStride) < nch) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > kSpinLimit) {
          flag_error(la.d.error, kErrWait);
          ok = 0u;
          break;
        }
      }
      st_agent_u32(la.e.counters + bh * kCounterStride, 0u);  // every item of the head counted
      s_ok = ok;
    }
    __syncthreads();
    if (s_ok != 0u) select_item<GROUP>(la.e, b, h, plan, sm.e.tk);
  } else if (t < la.n_workers + la.n_heads + la.n_dec) {
    const uint32_t err0 = *la.d.error;
    const uint32_t u = t - la.n_workers - la.n_heads;
    // decode items per (sequence, block of GI query heads, chunk)
    const uint32_t bh = u / la.d.max_chunks, chunk = u % la.d.max_chunks;
    const uint32_t nblk = la.d.Hq / GI;
    const uint32_t b = bh / nblk, hq0 = (bh % nblk) * GI;
    if constexpr (SELF) {
      // start when the head's scoring workers start (their staggered
      // schedule; heads of later rounds: the last first-round start):
      // earlier, the head's decode items only add page-table loads and
      // polls to the memory traffic of the first heads' scoring (23.0 vs
      // 24.15 us per layer at config 2)
      const uint32_t first_round = (la.n_workers - 1u) / la.est_chunks;
      const uint32_t bkv = b * la.d.Hkv + hq0 / GROUP;  // the (sequence, kv head)
      const uint32_t unit = bkv / HPI;                   // its scoring unit
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      sleep_until(t0, (uint64_t)(unit < first_round ? unit : first_round) * la.stagger_ps);
      TL(kTlStaggerDone);
      decode_item<true, QUEST, true, GI, GROUP == 1>(la.d, b, hq0, chunk, sm.d, &la.e, &sm.e.tk,
                                                     &s_err, err0);
    } else {
      decode_item<true, QUEST, false, GI, GROUP == 1>(la.d, b, hq0, chunk, sm.d, nullptr, nullptr,
                                                      &s_err, err0);
    }
  }
}

// grid-stride: a workspace of 16 GiB or more holds 2^32 words, more than one
// dispatch's 32-bit work-item count
__global__ void fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// ---------------------------------------------------------------- launchers

hipError_t launch_estimate(const EstimateArgs& a, uint32_t batch, uint32_t max_pages,
                           hipStream_t s) {
  const bool fused = a.sel != nullptr;
  const uint32_t ppb = est_kernel_block_pages_of(a.Hq / a.Hkv, fused);
  dim3 grid((max_pages + ppb - 1u) / ppb, a.Hkv, batch);
  switch (a.Hq / a.Hkv) {
#define AOAKV_EST(G)                                                                   \
  case G:                                                                              \
    if (fused) hipLaunchKernelGGL((estimate_kernel<G, true>), grid, dim3(kThreads), 0, s, a); \
    else hipLaunchKernelGGL((estimate_kernel<G, false>), grid, dim3(kThreads), 0, s, a);      \
    break;
    AOAKV_EST(1)
    AOAKV_EST(2)
    AOAKV_EST(4)
    AOAKV_EST(8)
#undef AOAKV_EST
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_layer(const LayerArgs& la, hipStream_t s) {
  if ((uint64_t)la.n_workers + la.n_heads + la.n_dec > layer_max_workgroups())
    return hipErrorInvalidConfiguration;
  const uint32_t grid = la.n_workers + la.n_heads + la.n_dec;
  const bool quest = (la.e.flags & kFlagQuestKernel) != 0u;
  const bool self = la.self_select != 0u;
  const bool grouped = la.d.heads_per_item > 1u;
  if (la.score_heads == 2u) {  // NHD head pairs (GROUP 1, score words)
    if (la.e.Hq != la.e.Hkv || la.e.Hkv % 2u != 0u || la.e.hscore == nullptr)
      return hipErrorInvalidValue;
    if (self && quest) hipLaunchKernelGGL((layer_kernel<1, true, true, 1, 2>), dim3(grid), dim3(kThreads), 0, s, la);
    else if (self) hipLaunchKernelGGL((layer_kernel<1, false, true, 1, 2>), dim3(grid), dim3(kThreads), 0, s, la);
    else if (quest) hipLaunchKernelGGL((layer_kernel<1, true, false, 1, 2>), dim3(grid), dim3(kThreads), 0, s, la);
    else hipLaunchKernelGGL((layer_kernel<1, false, false, 1, 2>), dim3(grid), dim3(kThreads), 0, s, la);
    return hipGetLastError();
  }
  switch (la.e.Hq / la.e.Hkv) {
#define AOAKV_LAYER_GI(G, GI)                                                                        \
  if (self && quest) hipLaunchKernelGGL((layer_kernel<G, true, true, GI>), dim3(grid), dim3(kThreads), 0, s, la);   \
  else if (self) hipLaunchKernelGGL((layer_kernel<G, false, true, GI>), dim3(grid), dim3(kThreads), 0, s, la);      \
  else if (quest) hipLaunchKernelGGL((layer_kernel<G, true, false, GI>), dim3(grid), dim3(kThreads), 0, s, la);     \
  else hipLaunchKernelGGL((layer_kernel<G, false, false, GI>), dim3(grid), dim3(kThreads), 0, s, la);
#define AOAKV_LAYER(G)                 \
  case G:                              \
    if (grouped) {                     \
      AOAKV_LAYER_GI(G, G)             \
    } else {                           \
      AOAKV_LAYER_GI(G, 1)             \
    }                                  \
    break;
    case 1: AOAKV_LAYER_GI(1, 1) break;
    AOAKV_LAYER(2)
    AOAKV_LAYER(4)
    AOAKV_LAYER(8)
#undef AOAKV_LAYER
#undef AOAKV_LAYER_GI
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

uint64_t layer_max_workgroups() { return 0xFFFFFFFFull / (uint64_t)kThreads; }

uint32_t est_chunks(uint32_t max_pages, uint32_t group) {
  const uint32_t n = est_block_pages_of(group);
  return (max_pages + n - 1u) / n;
}

hipError_t launch_topk(const TopkArgs& a, uint32_t batch, hipStream_t s) {
  hipLaunchKernelGGL(topk_kernel, dim3(a.Hkv, batch), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, uint32_t batch, hipStream_t s,
                         const EstimateArgs* self) {
  // one workgroup per (chunk, block of heads_per_item query heads, sequence)
  const uint32_t gi = a.heads_per_item > 1u ? a.Hq / a.Hkv : 1u;
  dim3 grid(a.max_chunks, a.Hq / gi, batch);
  const bool quest = (a.flags & kFlagQuestKernel) != 0u;
  const EstimateArgs e = self != nullptr ? *self : EstimateArgs{};
  switch (gi) {
#define AOAKV_DEC_S(G, ST)                                                                    \
  if (self != nullptr) {                                                                      \
    if (quest) hipLaunchKernelGGL((decode_kernel<true, G, true, ST>), grid, dim3(kThreads), 0, s, a, e); \
    else hipLaunchKernelGGL((decode_kernel<false, G, true, ST>), grid, dim3(kThreads), 0, s, a, e);      \
  } else if (quest) {                                                                         \
    hipLaunchKernelGGL((decode_kernel<true, G, false, ST>), grid, dim3(kThreads), 0, s, a, e);  \
  } else {                                                                                    \
    hipLaunchKernelGGL((decode_kernel<false, G, false, ST>), grid, dim3(kThreads), 0, s, a, e); \
  }
#define AOAKV_DEC(G)   \
  case G:              \
    AOAKV_DEC_S(G, false) \
    break;
    case 1:  // without GQA each page's K/V has one reader: streamed
      if (a.Hq == a.Hkv) {
        AOAKV_DEC_S(1, true)
      } else {
        AOAKV_DEC_S(1, false)
      }
      break;
    AOAKV_DEC(2)
    AOAKV_DEC(4)
    AOAKV_DEC(8)
#undef AOAKV_DEC
#undef AOAKV_DEC_S
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256 < 65536u ? (n + 255) / 256 : 65536u;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

uint32_t decode_chunks(uint32_t max_sel_pages) {
  return (max_sel_pages + kDecPagesPerBlock - 1) / kDecPagesPerBlock;
}
uint32_t partial_stride() { return kPartialStride; }
uint32_t decode_max_chunks() { return kMergeMaxChunks; }
uint32_t topk_max_pages() { return kTopkMaxPages; }
uint32_t fused_topk_max_pages() { return kFusedTopkMaxPages; }
// Scoring workgroups of the one-launch layer.  Items are scored head by head
// in rounds of n_workers; the heads of the last round finish last and their
// top-k, gather and merge are exposed, so the last round is kept to about 2
// heads.  Measured at config 2 (32 heads x 16 items, staggered start, score
// handoff words), us per layer by workers: 416: 23.41, 448: 23.32, 464:
// 23.24, 480: 23.16, 496: 24.01, 512: 23.71.  Between 256 (one per CU) and
// 480 (with the 32 top-k and 512 decode workgroups of config 2, all 1024
// workgroups that four per CU allow are resident together).  With at most
// kFewHeads (sequence, kv head) pairs, every item has a worker: a second
// round would hold a quarter of the heads (GQA, 32 query / 8 kv heads, 64
// items per head: 384 workers 15.8 us, 512 workers 15.4).
constexpr uint32_t kFewHeads = 8u;
uint32_t layer_score_workers(uint32_t n_est, uint32_t est_chunks) {
  if (n_est <= 256u) return n_est;
  if (n_est <= 512u && n_est / est_chunks <= kFewHeads) return n_est;
  const uint32_t last_round = 2u * est_chunks;
  uint32_t w = n_est > last_round ? n_est - last_round : 256u;
  w = w < 256u ? 256u : w;
  return w > 480u ? 480u : w;
}
// The scoring workers of the first round would otherwise issue all their
// loads at once, and HBM would finish every head's chunks at about the same
// time, late (a head is done when its last chunk is).  Starting head h's
// workers h * stagger in, a little faster than HBM streams one head's
// metadata (est_chunks * 128 pages * 514 B at kStreamBytesPerNs, so the
// memory queue never runs dry), finishes the heads one after another, so the
// top-k, gathers and merge of the first heads overlap the scoring of the
// later ones.  Timed in wall time (s_memrealtime), not core cycles, so the
// offset holds whatever the clock.  Config 2 (16 chunks per head: 1.05 MB),
// us per layer by bytes per ns: 5600: 24.06, 6100: 23.69, 6600: 23.35-23.39,
// 7100: 23.20-23.26, 7600: 23.31, 8200: 23.49, 9000: 23.85 (the former
// core-cycle stagger at its best, 376 cycles per head: 23.26).  Since the
// metadata and K/V stream with non-temporal loads (they reach HBM faster),
// 8,500 B/ns: 6,000 21.28, 7,100 20.52-20.56, 7,600 20.32-20.35, 8,000
// 20.21-20.25, 8,500 20.22-20.24, 9,000 20.24-20.27, 10,500 20.38-20.40
// (480 workers; 448: 20.81, 512: 20.22-20.25 at 8,500).  With at most
// kFewHeads heads every head starts at once: their metadata is a short
// stream whose heads all end in the same round (GQA above with 512 workers:
// no stagger 15.1 us, 7,100 B/ns 15.4, 14,000 B/ns 15.4).
uint32_t layer_stagger_ps(uint32_t est_chunks, uint32_t group, uint32_t heads) {
  if (heads <= kFewHeads) return 0u;
  const uint64_t chunk_bytes = est_block_pages_of(group) * (2u * kHeadDim * 2u + 2u);
  constexpr uint64_t kStreamBytesPerNs = 8500u;
  return (uint32_t)((uint64_t)est_chunks * chunk_bytes * 1000u / kStreamBytesPerNs);
}
uint32_t counter_stride() { return kCounterStride; }
// Workgroups of the self-selecting layer kernel one CU holds at once (its LDS
// and registers decide); 0 if the runtime cannot tell.
uint32_t layer_self_blocks_per_cu(uint32_t group, uint32_t heads_per_item, uint32_t score_heads) {
  int n = 0;
  hipError_t e = hipErrorInvalidValue;
  const bool gr = heads_per_item > 1u;
#define AOAKV_OCC(G, GI) \
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, layer_kernel<G, false, true, GI>, kThreads, 0)
  switch (group) {
    case 1:
      if (score_heads == 2u)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, layer_kernel<1, false, true, 1, 2>,
                                                         kThreads, 0);
      else
        AOAKV_OCC(1, 1);
      break;
    case 2: if (gr) AOAKV_OCC(2, 2); else AOAKV_OCC(2, 1); break;
    case 4: if (gr) AOAKV_OCC(4, 4); else AOAKV_OCC(4, 1); break;
    case 8: if (gr) AOAKV_OCC(8, 8); else AOAKV_OCC(8, 1); break;
    default: break;
  }
#undef AOAKV_OCC
  if (e != hipSuccess || n < 0) return 0u;
  return (uint32_t)n;
}

}  // namespace aoakv

#ifdef AOAKV_TIMELINE
// Profiling build only (not declared in aoakv.h): read back the phase
// timestamps of the last instrumented launch ([4096 workgroups][kTlEvents]
// uint64, synchronizing), or clear them.
extern "C" int aoakv_timeline_read(void* host, size_t bytes) {
  if (bytes > sizeof(aoakv::g_tl)) bytes = sizeof(aoakv::g_tl);
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(aoakv::g_tl), bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" int aoakv_timeline_clear() {
  static unsigned long long zero[aoakv::kTlMaxWg][aoakv::kTlEvents];
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(aoakv::g_tl), zero, sizeof(zero), 0,
                                hipMemcpyHostToDevice);
}
extern "C" int aoakv_timeline_events() { return aoakv::kTlEvents; }
#endif
