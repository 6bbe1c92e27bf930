// Kernel argument blocks and launchers shared by the HIP translation units
// and the C ABI (capi.cpp).
#pragma once

#include "device.hpp"

namespace aoakv {

// Per-head arrival counters sit one 128-byte line apart: counters sharing a
// line slow each other's atomics and polls.
constexpr uint32_t kCounterStride = 32;

// Bits of the workspace error word (32-bit word 2 of a workspace):
//   kErrWait       a bounded wait of the one-launch layer gave up; its output
//                  is invalid and handoff words may be left set
//   kErrTruncated  a sequence's device page table holds more pages than the
//                  call was sized for (max_pages, a score or selection row,
//                  or a kernel limit); that sequence was computed on a
//                  truncated page list
constexpr uint32_t kErrWait = 1u;
constexpr uint32_t kErrTruncated = 2u;
// Workspace word that holds the error bits.
constexpr uint32_t kErrWord = 2u;

// Sets error bits (a no-op for entry points without a workspace).
__device__ inline void flag_error(uint32_t* error, uint32_t bits) {
  if (error != nullptr) atomicOr(error, bits);
}

// Selected pages per decode chunk of the generic kernels (as the tuned
// kernels' 8): the workspace's partials are laid out per chunk of 8.
constexpr uint32_t kGenChunkPages = 8u;

// Head dims the library takes: the tuned kernels are for kHeadDim (with
// kPageSize); 64 and 256, and other page sizes up to kMaxPageSize, run the
// kernels of generic.hip.
constexpr int kMaxHeadDim = 256;
constexpr uint32_t kMaxPageSize = 32;
inline bool tuned_shape(uint32_t head_dim, uint32_t page_size) {
  return head_dim == (uint32_t)kHeadDim && page_size == (uint32_t)kPageSize;
}
// The MFMA prefill takes head dims 64, 128 and 256 with page sizes 1, 2, 4,
// 8, 16 and 32: a wave's 16 key rows of a tile lie in 16 / S pages, or half
// of one.
inline bool prefill_tuned_shape(uint32_t head_dim, uint32_t page_size) {
  return (head_dim == 64u || head_dim == (uint32_t)kHeadDim || head_dim == 256u) &&
         page_size != 0u && page_size <= 32u && (page_size & (page_size - 1u)) == 0u;
}

// RoPE frequencies f_i = rcp_scale * rcp_theta^(2i / D), i < D / 2: fixed by
// (rope_scale, rope_theta, D), so computed once on the host (rope_freqs) and
// passed with the launch instead of per lane on the device.
struct RopeFreqs {
  float f[kMaxHeadDim / 2];
};
RopeFreqs rope_freqs(float rope_scale, float rope_theta, uint32_t head_dim = kHeadDim);

struct AppendPrefillArgs {
  const f16* k;            // [N, H, D]
  const f16* v;            // [N, H, D]
  f16* kv;                 // paged cache of the layer
  const int32_t* kv_indices;
  f16* meta;               // metadata cache of the layer
  const int32_t* meta_indices;
  f16* v_log_norm;         // [max_pages, H]
  f16* v_mean;             // [max_pages, H, D]
  uint32_t N, H, S, num_pages, last_page_len, first_page;
  PageGeom g;
};

struct AppendDecodeArgs {
  f16* k;        // [B, H, D] (rotated in place when rope)
  const f16* v;
  f16* kv;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_last_page_len;
  f16* meta;
  const int32_t* meta_indptr;
  const int32_t* meta_indices;
  f16* v_log_norm;
  f16* v_mean;
  uint32_t H, S;
  PageGeom g;
  // fused RoPE (rope != 0): q [B, Hq, D] and k rotated in place at each
  // sequence's new position, k stored rotated
  uint32_t rope;
  f16* q;
  uint32_t Hq;
  RopeFreqs rope_f;
};

struct RopeArgs {
  f16* q;  // [N, Hq, D]
  f16* k;  // [N, Hkv, D]
  uint32_t N, past, Hq, Hkv;
  RopeFreqs rope_f;
};

struct EstimateArgs {
  const f16* q;  // [B, Hq, D]
  float* scores; // [B, Hkv, score_stride]
  uint32_t score_stride;
  const f16* meta;
  const int32_t* meta_indptr;
  const int32_t* meta_indices;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_last_page_len;
  const f16* v_log_norm;  // [max_pages, Hkv]
  uint32_t Hq, Hkv, S, flags;
  uint32_t max_pages;  // pages the grid covers per (sequence, head)
  PageGeom g;
  // fused top-k (sel == nullptr: scores only)
  int32_t* sel;
  uint32_t sel_stride;
  uint32_t token_budget;
  const int32_t* token_budgets;
  uint32_t* counters;  // [B * Hkv]
  // single launch only: the selection again, per query head, as page + 1
  // (0 = not yet written), for the decode items of the same launch
  uint32_t* hsel;      // [B, Hq, hsel_stride] or nullptr: a copy per decode item
  uint32_t hsel_stride;
  uint32_t hsel_gi;    // query heads per decode item (rows b * Hq + hq0 are read)
  // single launch only, optional: the scores again as handoff words (bits +
  // 1, 0 = not yet written), [B, Hkv, hscore_copies, hscore_stride]; the
  // top-k polls these instead of an arrival counter and clears them.  With
  // self-selecting decode items, one copy per decode block of the group
  // (group / heads_per_item), each read and cleared by that block's items
  uint32_t* hscore;
  uint32_t hscore_stride;
  uint32_t hscore_copies;
  uint32_t* error;  // workspace error word, or nullptr (no workspace)
};

struct TopkArgs {
  const float* scores;
  uint32_t score_stride;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_last_page_len;
  uint32_t token_budget;
  const int32_t* token_budgets;
  int32_t* sel;
  uint32_t sel_stride;
  uint32_t Hkv, S, flags;
  uint32_t* error;  // workspace error word, or nullptr (no workspace)
};

struct DecodeArgs {
  const f16* q;  // [B, Hq, D]
  f16* o;        // [B, Hq, D]
  const f16* kv;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_last_page_len;
  const int32_t* sel;  // [B, Hkv, sel_stride] physical ids, or nullptr (dense)
  uint32_t sel_stride;
  uint32_t token_budget;
  const int32_t* token_budgets;
  float* partial;      // [B*Hq, max_chunks, kPartialStride]
  uint32_t* counters;  // [B*Hq]
  uint32_t Hq, Hkv, S, max_chunks;
  uint32_t max_pages;  // pages per sequence the call is sized for (as the scoring's)
  uint32_t flags;      // kFlagQuestKernel: the quest_kernel selection convention
  // query heads per workgroup: 1 (each query head its own workgroups) or
  // Hq / Hkv (one workgroup per kv head serves its whole group)
  uint32_t heads_per_item;
  PageGeom g;
  // single launch only: handoff buffers whose words hold value + 1 (0 = not
  // yet written); every word is cleared again by its reader
  uint32_t* hsel;      // [B, Hq, hsel_stride] selection of this launch (row b * Hq + hq0)
  uint32_t hsel_stride;
  uint32_t* hpart;     // [B*Hq, max_chunks, kPartialStride] split-K partials
  uint32_t* error;     // workspace error word (kErrWait, kErrTruncated)
};

struct PrefillArgs {
  const f16* q;  // [Lq, Hq, D]
  f16* o;        // [Lq, Hq, D]
  const f16* kv;
  const int32_t* kv_indices;
  uint32_t H, L, Lq, causal;  // H: kv heads of the cache
  uint32_t Hq;                // query heads, a multiple of H
  float sm_scale;
  PageGeom g;
};

// One decode layer in one launch (see layer_kernel in decode.hip).
struct LayerArgs {
  EstimateArgs e;      // with sel / counters / hsel of the top-k
  DecodeArgs d;        // with hsel / hpart / error
  uint32_t n_est;      // scoring items: B * Hkv * est_chunks
  uint32_t est_chunks; // scoring items (128 / group pages each) per (sequence, kv head)
  uint32_t n_workers;  // scoring workgroups (<= n_est), items taken round-robin
  uint32_t n_heads;    // top-k workgroups: B * Hkv
  uint32_t n_dec;      // decode items: B * (Hq / d.heads_per_item) * d.max_chunks
  uint32_t stagger_ps; // wall time (ps) between the scoring starts of consecutive heads
  uint32_t self_select;  // decode items run their kv head's top-k themselves (n_heads = 0)
  uint32_t score_heads;  // kv heads per scoring item: 1, or 2 (NHD pairs, GROUP 1, score words)
};

hipError_t launch_append_prefill(const AppendPrefillArgs& a, hipStream_t s);
hipError_t launch_append_decode(const AppendDecodeArgs& a, uint32_t batch, hipStream_t s);
hipError_t launch_rope(const RopeArgs& a, hipStream_t s);
hipError_t launch_estimate(const EstimateArgs& a, uint32_t batch, uint32_t max_pages,
                           hipStream_t s);
hipError_t launch_topk(const TopkArgs& a, uint32_t batch, hipStream_t s);
hipError_t launch_layer(const LayerArgs& la, hipStream_t s);
uint32_t est_chunks(uint32_t max_pages, uint32_t group);  // scoring items per (sequence, kv head)
uint64_t layer_max_workgroups();  // one-launch layer grid limit (32-bit work-item count)
// self: the decode items select for themselves from the scores of the
// previous launch (the scoring call's arguments, with sel / budgets / flags)
hipError_t launch_decode(const DecodeArgs& a, uint32_t batch, hipStream_t s,
                         const EstimateArgs* self = nullptr);
hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s);
hipError_t launch_prefill(const PrefillArgs& a, uint32_t page_size, uint32_t head_dim,
                          hipStream_t s);

// RMSNorm of `rows` fp16 rows of n elements (n a multiple of 8), one weight row.
struct RmsNormArgs {
  const f16* x;
  const f16* w;
  f16* out;
  uint32_t n;
  float eps;
};
hipError_t launch_rms_norm(const RmsNormArgs& a, uint32_t rows, hipStream_t s);
uint32_t decode_chunks(uint32_t max_sel_pages);
uint32_t partial_stride();
uint32_t decode_max_chunks();  // split-K chunks per head the merge holds
uint32_t topk_max_pages();     // pages per (sequence, head) top-k supports
uint32_t fused_topk_max_pages();  // ... and the fused estimate + top-k kernel
uint32_t layer_score_workers(uint32_t n_est, uint32_t est_chunks);  // one-launch layer scorers
uint32_t layer_stagger_ps(uint32_t est_chunks, uint32_t group, uint32_t heads);  // one-launch scoring start offset per head (ps)
uint32_t counter_stride();        // u32 words between per-head counters (one cache line each)
uint32_t layer_self_blocks_per_cu(uint32_t group, uint32_t heads_per_item, uint32_t score_heads);  // per CU

// generic.hip: the other head dims (64, 128, 256) and page sizes (1..32)
hipError_t launch_gen_append_prefill(const AppendPrefillArgs& a, uint32_t head_dim, hipStream_t s);
hipError_t launch_gen_append_decode(const AppendDecodeArgs& a, uint32_t batch, uint32_t head_dim,
                                    hipStream_t s);
hipError_t launch_gen_rope(const RopeArgs& a, uint32_t head_dim, hipStream_t s);
hipError_t launch_gen_estimate(const EstimateArgs& a, uint32_t batch, uint32_t max_pages,
                               uint32_t head_dim, hipStream_t s);
hipError_t launch_gen_decode(const DecodeArgs& a, uint32_t batch, uint32_t head_dim,
                             hipStream_t s);
hipError_t launch_gen_prefill(const PrefillArgs& a, uint32_t head_dim, hipStream_t s);

}  // namespace aoakv
