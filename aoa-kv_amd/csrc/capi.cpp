// extern "C" boundary of libaoakv.so (declared in include/aoakv.h).
//
// Each entry point validates its arguments on the host (shapes the kernels
// assume, null pointers, budgets), then launches on the caller's stream.
// Nothing here allocates device memory or synchronises.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/aoakv.h"
#include "kernels.hpp"

namespace aoakv {
RopeFreqs rope_freqs(float rope_scale, float rope_theta, uint32_t head_dim) {
  RopeFreqs r{};
  const float rcp_scale = 1.0f / rope_scale, rcp_theta = 1.0f / rope_theta;
  for (uint32_t i = 0; i < head_dim / 2u; ++i)
    r.f[i] = (float)((double)rcp_scale *
                     std::pow((double)rcp_theta, (double)(2u * i) / (double)head_dim));
  return r;
}
}  // namespace aoakv

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return AOAKV_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(AOAKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// Workgroups of the self-selecting one-launch layer the current device holds
// at once: CUs times the kernel's occupancy per CU (four at 36 KB of LDS and
// 112 VGPRs).  0 if the device cannot be queried.  Cached per device (benign
// races: every writer stores the same value).
uint32_t resident_layer_workgroups(uint32_t group, uint32_t heads_per_item, uint32_t score_heads) {
  static uint32_t cache[64][9];
  const uint32_t gi = score_heads == 2u ? 8u
                      : (group == 1u ? 0u : group == 2u ? 1u : group == 4u ? 2u : 3u) +
                            (heads_per_item > 1u ? 4u : 0u);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0u;
  if (cache[dev][gi] == 0u) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      return 0u;
    cache[dev][gi] =
        aoakv::layer_self_blocks_per_cu(group, heads_per_item, score_heads) * (uint32_t)cus;
  }
  return cache[dev][gi];
}

#define REQUIRE(cond, ...)                                  \
  do {                                                      \
    if (!(cond)) return fail(AOAKV_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// head_dim 64 / 128 / 256 (the reference's SWITCH_HEAD_DIM) and page sizes
// 1..32; (128, 16) runs the tuned kernels, the rest generic.hip's
int check_shape(uint32_t head_dim, uint32_t page_size, uint32_t layout, uint32_t num_heads) {
  if (head_dim != 64u && head_dim != 128u && head_dim != 256u)
    return fail(AOAKV_ERR_UNSUPPORTED, "head_dim %u unsupported (64, 128, 256)", head_dim);
  if (page_size == 0u || page_size > aoakv::kMaxPageSize)
    return fail(AOAKV_ERR_UNSUPPORTED, "page_size %u unsupported (1..%u)", page_size,
                aoakv::kMaxPageSize);
  if (layout > 1u) return fail(AOAKV_ERR_UNSUPPORTED, "layout %u unknown (0=NHD, 1=HND)", layout);
  if (num_heads == 0u || num_heads > 256u)
    return fail(AOAKV_ERR_UNSUPPORTED, "num_heads %u out of range [1, 256]", num_heads);
  return AOAKV_OK;
}

// Selection flags a scoring / top-k / decode entry point accepts.
constexpr uint32_t kSelectFlags =
    AOAKV_FLAG_VALUE_AWARE | AOAKV_FLAG_FIXED | AOAKV_FLAG_QUEST_KERNEL;

int check_flags(uint32_t flags, uint32_t allowed, const char* fn) {
  if (flags & ~allowed) return fail(AOAKV_ERR_INVALID, "%s: unknown flags 0x%x", fn, flags);
  if ((flags & AOAKV_FLAG_FIXED) && (flags & AOAKV_FLAG_QUEST_KERNEL))
    return fail(AOAKV_ERR_INVALID,
                "%s: AOAKV_FLAG_FIXED does not apply to AOAKV_FLAG_QUEST_KERNEL (the last page "
                "is always attended, no page is forced into the selection)",
                fn);
  return AOAKV_OK;
}

// Smallest selection row: the simulation's k is at least 3; the
// quest_kernel convention selects k - 1 >= 0 pages besides the last.
uint32_t min_sel_stride(uint32_t flags) { return (flags & AOAKV_FLAG_QUEST_KERNEL) ? 1u : 3u; }

// Pages one head attends at most: every page (dense), else the selection row
// (plus the last page with the quest_kernel convention), and with one token
// budget for every sequence no more than that budget selects at any length
// (num_selected_pages is monotone in the length and the page count).  The
// decode grid, its workspace regions and the one-launch selection handoff
// rows are sized by it, so a caller's selection buffer wider than the budget
// (one row per page of the cache) costs no idle workgroups.
uint32_t max_selected(const int32_t* sel_pages, uint32_t sel_stride, uint32_t token_budget,
                      const int32_t* token_budgets, uint32_t max_pages, uint32_t page_size,
                      uint32_t flags) {
  if (!sel_pages) return max_pages;
  const bool quest = (flags & AOAKV_FLAG_QUEST_KERNEL) != 0u;
  const uint32_t row = sel_stride + (quest ? 1u : 0u);
  uint32_t m = row < max_pages ? row : max_pages;
  if (!token_budgets) {
    const uint32_t k = aoakv::num_selected_pages(0xFFFFFFFFu, token_budget, page_size, max_pages,
                                                 quest ? aoakv::kFlagQuestKernel : 0u);
    m = k < m ? k : m;
  }
  return m;
}

int check_group(uint32_t hq, uint32_t hkv) {
  if (hkv == 0u || hq % hkv != 0u)
    return fail(AOAKV_ERR_INVALID, "num_qo_heads %u not a multiple of num_kv_heads %u", hq, hkv);
  uint32_t g = hq / hkv;
  if (g != 1u && g != 2u && g != 4u && g != 8u)
    return fail(AOAKV_ERR_UNSUPPORTED, "GQA group size %u unsupported (1, 2, 4, 8)", g);
  return AOAKV_OK;
}

struct Workspace {
  uint32_t* ctl;  // word 2 (kErrWord): error bits kErrWait, kErrTruncated
  uint32_t* est_counters;
  uint32_t* dec_counters;
  float* partial;
  uint32_t* hsel;
  uint32_t* hpart;
  size_t bytes;
};

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// the control words at the start of every workspace (64 u32)
constexpr size_t kCtlBytes = 256;

// [ctl: 64 u32][est counters: B*Hkv lines][dec counters: B*Hq lines]
// [partials: B*Hq*chunks*stride f32][hsel: B*Hq*max_sel u32]
// [hpart: B*Hq*chunks*stride u32]; stride = head_dim + 4 (o, m, l, pad),
// chunks of 8 selected pages; every region 256-byte aligned.  The
// control words sit at offset 0 so a caller can read the error flag (word
// 2) without knowing the shapes.  All of it starts zeroed
// (aoakv_workspace_init) and every launch leaves all of it zeroed again
// (the offsets depend on the call's selection size, so a region that must
// start at zero in one call can lie where another call kept other data).
size_t ws_layout(uint32_t B, uint32_t hq, uint32_t hkv, uint32_t max_sel_pages, uint32_t head_dim,
                 void* base, Workspace* w) {
  const size_t part =
      (size_t)B * hq * aoakv::decode_chunks(max_sel_pages) * (head_dim + 4u) * 4u;
  const size_t off_est = kCtlBytes;
  const size_t cnt = (size_t)aoakv::counter_stride() * 4u;  // bytes per counter
  const size_t off_dec = off_est + round_up((size_t)B * hkv * cnt, 256);
  const size_t off_part = off_dec + round_up((size_t)B * hq * cnt, 256);
  const size_t off_hsel = off_part + round_up(part, 256);
  const size_t off_hpart = off_hsel + round_up((size_t)B * hq * max_sel_pages * 4u, 256);
  const size_t total = off_hpart + round_up(part, 256);
  if (w) {
    char* c = static_cast<char*>(base);
    w->ctl = reinterpret_cast<uint32_t*>(c);
    w->est_counters = reinterpret_cast<uint32_t*>(c + off_est);
    w->dec_counters = reinterpret_cast<uint32_t*>(c + off_dec);
    w->partial = reinterpret_cast<float*>(c + off_part);
    w->hsel = reinterpret_cast<uint32_t*>(c + off_hsel);
    w->hpart = reinterpret_cast<uint32_t*>(c + off_hpart);
    w->bytes = total;
  }
  return total;
}

// Scores + top-k: one fused launch when every sequence fits the fused
// kernel's top-k, else scores then the standalone top-k kernel (always so
// for the shapes of generic.hip).
int launch_estimate_topk(aoakv::EstimateArgs ea, const Workspace& w, int32_t* sel_pages,
                         uint32_t sel_stride, uint32_t token_budget, const int32_t* token_budgets,
                         uint32_t batch_size, uint32_t max_pages, uint32_t head_dim,
                         uint32_t page_size, uint32_t flags, hipStream_t s) {
  const bool tuned = aoakv::tuned_shape(head_dim, page_size);
  if (tuned && max_pages <= aoakv::fused_topk_max_pages()) {
    ea.sel = sel_pages;
    ea.sel_stride = sel_stride;
    ea.token_budget = token_budget;
    ea.token_budgets = token_budgets;
    ea.counters = w.est_counters;
    return hip_status(aoakv::launch_estimate(ea, batch_size, max_pages, s), "estimate_topk");
  }
  if (int e = hip_status(tuned ? aoakv::launch_estimate(ea, batch_size, max_pages, s)
                               : aoakv::launch_gen_estimate(ea, batch_size, max_pages, head_dim, s),
                         "estimate"))
    return e;
  aoakv::TopkArgs ta{};
  ta.scores = ea.scores;
  ta.score_stride = ea.score_stride;
  ta.kv_indptr = ea.kv_indptr;
  ta.kv_indices = ea.kv_indices;
  ta.kv_last_page_len = ea.kv_last_page_len;
  ta.token_budget = token_budget;
  ta.token_budgets = token_budgets;
  ta.sel = sel_pages;
  ta.sel_stride = sel_stride;
  ta.Hkv = ea.Hkv;
  ta.S = page_size;
  ta.flags = flags & kSelectFlags;
  ta.error = ea.error;
  return hip_status(aoakv::launch_topk(ta, batch_size, s), "topk");
}

// ---------------------------------------------------------------- no-allocation scratch
// aoakv_sparse_decode_layer_noalloc's workspace: a file-scope device array,
// one per GPU the library runs on, held until the process ends.  Host code
// never uses the array's name as an address (on the host it is only a
// stand-in symbol): the device address comes from hipGetSymbolAddress, once
// per device with that device current, and is kept per device.  The array
// starts zeroed (module load), and the two-launch kernels that use it leave
// its counters and partials at zero after every call, so no call clears it.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];

// The scratch array's device address on the current device, resolved on the
// first call per device (aoakv_noalloc_init makes that call outside any
// stream capture).  `who` names the entry point in error messages.
int scratch_for_current_device(void** out, const char* who) {
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
    return fail(AOAKV_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= 64)
    return fail(AOAKV_ERR_UNSUPPORTED, "%s: device %d out of range", who, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess || !p)
      return fail(AOAKV_ERR_HIP, "%s: hipGetSymbolAddress: %s", who, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AOAKV_OK;
}

}  // namespace

extern "C" {

const char* aoakv_last_error(void) { return g_err.c_str(); }

const char* aoakv_version(void) { return "aoakv-mi355x 0.1 (gfx950)"; }

int aoakv_append_kv_cache_prefill(const void* k, const void* v, uint32_t num_new_tokens,
                                  void* kv_data, const int32_t* kv_indices,
                                  uint32_t num_kv_pages, uint32_t kv_last_page_len,
                                  void* metadata_data, const int32_t* metadata_indices,
                                  void* v_log_norm, void* v_mean, uint32_t num_heads,
                                  uint32_t head_dim, uint32_t page_size, uint32_t layout,
                                  void* stream) {
  if (int e = check_shape(head_dim, page_size, layout, num_heads)) return e;
  REQUIRE(k && v && kv_data && kv_indices && metadata_data && metadata_indices && v_log_norm &&
              v_mean,
          "append_kv_cache_prefill: null pointer argument");
  REQUIRE(num_kv_pages >= 1u, "append_kv_cache_prefill: num_kv_pages must be >= 1");
  REQUIRE(kv_last_page_len >= 1u && kv_last_page_len <= page_size,
          "append_kv_cache_prefill: kv_last_page_len %u not in [1, %u]", kv_last_page_len,
          page_size);
  const uint64_t L = (uint64_t)(num_kv_pages - 1u) * page_size + kv_last_page_len;
  REQUIRE(num_new_tokens >= 1u && num_new_tokens <= L,
          "append_kv_cache_prefill: %u new tokens but the cache holds %llu", num_new_tokens,
          (unsigned long long)L);
  aoakv::AppendPrefillArgs a{};
  a.k = static_cast<const aoakv::f16*>(k);
  a.v = static_cast<const aoakv::f16*>(v);
  a.kv = static_cast<aoakv::f16*>(kv_data);
  a.kv_indices = kv_indices;
  a.meta = static_cast<aoakv::f16*>(metadata_data);
  a.meta_indices = metadata_indices;
  a.v_log_norm = static_cast<aoakv::f16*>(v_log_norm);
  a.v_mean = static_cast<aoakv::f16*>(v_mean);
  a.N = num_new_tokens;
  a.H = num_heads;
  a.S = page_size;
  a.num_pages = num_kv_pages;
  a.last_page_len = kv_last_page_len;
  a.g = aoakv::make_geom(layout, num_heads, page_size, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(aoakv::tuned_shape(head_dim, page_size)
                        ? aoakv::launch_append_prefill(a, s)
                        : aoakv::launch_gen_append_prefill(a, head_dim, s),
                    "append_kv_cache_prefill");
}

int aoakv_append_kv_cache_decode(const void* k, const void* v, uint32_t batch_size,
                                 void* kv_data, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                 void* metadata_data, const int32_t* metadata_indptr,
                                 const int32_t* metadata_indices, void* v_log_norm,
                                 void* v_mean, uint32_t num_heads, uint32_t head_dim,
                                 uint32_t page_size, uint32_t layout, void* stream) {
  if (int e = check_shape(head_dim, page_size, layout, num_heads)) return e;
  REQUIRE(k && v && kv_data && kv_indptr && kv_indices && kv_last_page_len && metadata_data &&
              metadata_indptr && metadata_indices && v_log_norm && v_mean,
          "append_kv_cache_decode: null pointer argument");
  REQUIRE(batch_size >= 1u && batch_size <= 65535u,
          "append_kv_cache_decode: batch_size %u out of range", batch_size);
  aoakv::AppendDecodeArgs a{};
  // k is only read without RoPE
  a.k = static_cast<aoakv::f16*>(const_cast<void*>(k));
  a.v = static_cast<const aoakv::f16*>(v);
  a.kv = static_cast<aoakv::f16*>(kv_data);
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_last_page_len = kv_last_page_len;
  a.meta = static_cast<aoakv::f16*>(metadata_data);
  a.meta_indptr = metadata_indptr;
  a.meta_indices = metadata_indices;
  a.v_log_norm = static_cast<aoakv::f16*>(v_log_norm);
  a.v_mean = static_cast<aoakv::f16*>(v_mean);
  a.H = num_heads;
  a.S = page_size;
  a.g = aoakv::make_geom(layout, num_heads, page_size, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(aoakv::tuned_shape(head_dim, page_size)
                        ? aoakv::launch_append_decode(a, batch_size, s)
                        : aoakv::launch_gen_append_decode(a, batch_size, head_dim, s),
                    "append_kv_cache_decode");
}

// RoPE factors as the reference passes them (rope_scale, rope_theta; the
// kernel uses their reciprocals, decode_page.cuh:855-856).
static int check_rope(float rope_scale, float rope_theta, const char* fn) {
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f) || !std::isfinite(rope_scale) ||
      !std::isfinite(rope_theta))
    return fail(AOAKV_ERR_INVALID, "%s: rope_scale %g / rope_theta %g must be positive", fn,
                (double)rope_scale, (double)rope_theta);
  return AOAKV_OK;
}

int aoakv_rms_norm_forward(const void* x, const void* w, void* out, uint32_t rows, uint32_t n,
                           float epsilon, void* stream) {
  REQUIRE(x && w && out, "rms_norm_forward: null pointer argument");
  REQUIRE(rows >= 1u, "rms_norm_forward: rows must be >= 1");
  REQUIRE(n >= 8u && n <= 65536u && n % 8u == 0u,
          "rms_norm_forward: n = %u must be a multiple of 8 in [8, 65536]", n);
  REQUIRE(epsilon >= 0.f, "rms_norm_forward: epsilon must be >= 0");
  aoakv::RmsNormArgs a{};
  a.x = static_cast<const aoakv::f16*>(x);
  a.w = static_cast<const aoakv::f16*>(w);
  a.out = static_cast<aoakv::f16*>(out);
  a.n = n;
  a.eps = epsilon;
  return hip_status(aoakv::launch_rms_norm(a, rows, static_cast<hipStream_t>(stream)),
                    "rms_norm_forward");
}

int aoakv_apply_rope_in_place(void* q, void* k, uint32_t seq_len, uint32_t past_kv_len,
                              uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                              float rope_scale, float rope_theta, void* stream) {
  if (int e = check_shape(head_dim, aoakv::kPageSize, 0u, num_qo_heads)) return e;
  REQUIRE(q && k, "apply_rope_in_place: null pointer argument");
  REQUIRE(num_kv_heads >= 1u && num_kv_heads <= 256u,
          "apply_rope_in_place: num_kv_heads %u out of range [1, 256]", num_kv_heads);
  REQUIRE(seq_len <= 0x7FFFFFFFu && (uint64_t)past_kv_len + seq_len <= (1ull << 24),
          "apply_rope_in_place: positions up to %llu exceed 2^24 (fp32 positions)",
          (unsigned long long)past_kv_len + seq_len);
  if (int e = check_rope(rope_scale, rope_theta, "apply_rope_in_place")) return e;
  aoakv::RopeArgs a{};
  a.q = static_cast<aoakv::f16*>(q);
  a.k = static_cast<aoakv::f16*>(k);
  a.N = seq_len;
  a.past = past_kv_len;
  a.Hq = num_qo_heads;
  a.Hkv = num_kv_heads;
  a.rope_f = aoakv::rope_freqs(rope_scale, rope_theta, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(head_dim == (uint32_t)aoakv::kHeadDim ? aoakv::launch_rope(a, s)
                                                          : aoakv::launch_gen_rope(a, head_dim, s),
                    "apply_rope_in_place");
}

int aoakv_rope_append_kv_cache_decode(void* q, void* k, const void* v, uint32_t batch_size,
                                      uint32_t num_qo_heads, void* kv_data,
                                      const int32_t* kv_indptr, const int32_t* kv_indices,
                                      const int32_t* kv_last_page_len, void* metadata_data,
                                      const int32_t* metadata_indptr,
                                      const int32_t* metadata_indices, void* v_log_norm,
                                      void* v_mean, uint32_t num_heads, uint32_t head_dim,
                                      uint32_t page_size, uint32_t layout, float rope_scale,
                                      float rope_theta, void* stream) {
  if (int e = check_shape(head_dim, page_size, layout, num_heads)) return e;
  REQUIRE(q, "rope_append_kv_cache_decode: null pointer argument");
  REQUIRE(num_qo_heads >= 1u && num_qo_heads <= 256u,
          "rope_append_kv_cache_decode: num_qo_heads %u out of range [1, 256]", num_qo_heads);
  if (int e = check_rope(rope_scale, rope_theta, "rope_append_kv_cache_decode")) return e;
  REQUIRE(k && v && kv_data && kv_indptr && kv_indices && kv_last_page_len && metadata_data &&
              metadata_indptr && metadata_indices && v_log_norm && v_mean,
          "rope_append_kv_cache_decode: null pointer argument");
  REQUIRE(batch_size >= 1u && batch_size <= 65535u,
          "rope_append_kv_cache_decode: batch_size %u out of range", batch_size);
  aoakv::AppendDecodeArgs a{};
  a.k = static_cast<aoakv::f16*>(k);
  a.v = static_cast<const aoakv::f16*>(v);
  a.kv = static_cast<aoakv::f16*>(kv_data);
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_last_page_len = kv_last_page_len;
  a.meta = static_cast<aoakv::f16*>(metadata_data);
  a.meta_indptr = metadata_indptr;
  a.meta_indices = metadata_indices;
  a.v_log_norm = static_cast<aoakv::f16*>(v_log_norm);
  a.v_mean = static_cast<aoakv::f16*>(v_mean);
  a.H = num_heads;
  a.S = page_size;
  a.g = aoakv::make_geom(layout, num_heads, page_size, head_dim);
  a.rope = 1u;
  a.q = static_cast<aoakv::f16*>(q);
  a.Hq = num_qo_heads;
  a.rope_f = aoakv::rope_freqs(rope_scale, rope_theta, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(aoakv::tuned_shape(head_dim, page_size)
                        ? aoakv::launch_append_decode(a, batch_size, s)
                        : aoakv::launch_gen_append_decode(a, batch_size, head_dim, s),
                    "rope_append_kv_cache_decode");
}

static int fill_estimate(aoakv::EstimateArgs& a, const void* q, float* scores,
                         uint32_t score_stride, const void* metadata_data,
                         const int32_t* metadata_indptr, const int32_t* metadata_indices,
                         const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, const void* v_log_norm,
                         uint32_t batch_size, uint32_t max_pages, uint32_t num_qo_heads,
                         uint32_t num_kv_heads, uint32_t head_dim, uint32_t page_size,
                         uint32_t layout, uint32_t flags) {
  if (int e = check_shape(head_dim, page_size, layout, num_qo_heads)) return e;
  if (int e = check_group(num_qo_heads, num_kv_heads)) return e;
  REQUIRE(q && scores && metadata_data && metadata_indptr && metadata_indices && kv_indptr &&
              kv_indices && kv_last_page_len,
          "estimate_attn_score: null pointer argument");
  REQUIRE(batch_size >= 1u && batch_size <= 65535u, "estimate_attn_score: bad batch_size %u",
          batch_size);
  if (int e = check_flags(flags, kSelectFlags | AOAKV_FLAG_SINGLE_LAUNCH, "estimate_attn_score"))
    return e;
  // the quest_kernel convention leaves the last page unscored
  const uint32_t row = (flags & AOAKV_FLAG_QUEST_KERNEL) ? max_pages - 1u : max_pages;
  REQUIRE(max_pages >= 1u && score_stride >= row && score_stride >= 1u,
          "estimate_attn_score: score_stride %u < %u scores per row", score_stride, row);
  REQUIRE(!(flags & AOAKV_FLAG_VALUE_AWARE) || v_log_norm,
          "estimate_attn_score: value-aware scoring needs v_log_norm");
  a.q = static_cast<const aoakv::f16*>(q);
  a.scores = scores;
  a.score_stride = score_stride;
  a.meta = static_cast<const aoakv::f16*>(metadata_data);
  a.meta_indptr = metadata_indptr;
  a.meta_indices = metadata_indices;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_last_page_len = kv_last_page_len;
  a.v_log_norm = static_cast<const aoakv::f16*>(v_log_norm);
  a.Hq = num_qo_heads;
  a.Hkv = num_kv_heads;
  a.S = page_size;
  a.flags = flags;
  a.max_pages = max_pages;
  a.g = aoakv::make_geom(layout, num_kv_heads, page_size, head_dim);
  return AOAKV_OK;
}

int aoakv_estimate_attn_score(const void* q, float* scores, uint32_t score_stride,
                              const void* metadata_data, const int32_t* metadata_indptr,
                              const int32_t* metadata_indices, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              const void* v_log_norm, uint32_t batch_size, uint32_t max_pages,
                              uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                              uint32_t page_size, uint32_t layout, uint32_t flags,
                              void* stream) {
  aoakv::EstimateArgs a{};
  if (int e = fill_estimate(a, q, scores, score_stride, metadata_data, metadata_indptr,
                            metadata_indices, kv_indptr, kv_indices, kv_last_page_len,
                            v_log_norm, batch_size, max_pages, num_qo_heads, num_kv_heads,
                            head_dim, page_size, layout, flags))
    return e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(aoakv::tuned_shape(head_dim, page_size)
                        ? aoakv::launch_estimate(a, batch_size, max_pages, s)
                        : aoakv::launch_gen_estimate(a, batch_size, max_pages, head_dim, s),
                    "estimate_attn_score");
}

int aoakv_topk_filtering(const float* scores, uint32_t score_stride,
                         const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, uint32_t token_budget,
                         const int32_t* token_budgets, int32_t* sel_pages, uint32_t sel_stride,
                         uint32_t batch_size, uint32_t num_kv_heads, uint32_t page_size,
                         uint32_t flags, uint32_t* error_word, void* stream) {
  REQUIRE(scores && kv_indptr && kv_indices && kv_last_page_len && sel_pages,
          "topk_filtering: null pointer argument");
  REQUIRE(page_size >= 1u && page_size <= aoakv::kMaxPageSize,
          "topk_filtering: page_size %u unsupported (1..%u)", page_size, aoakv::kMaxPageSize);
  REQUIRE(batch_size >= 1u && batch_size <= 65535u && num_kv_heads >= 1u &&
              num_kv_heads <= 65535u,
          "topk_filtering: bad batch_size %u / num_kv_heads %u", batch_size, num_kv_heads);
  if (int e = check_flags(flags, kSelectFlags, "topk_filtering")) return e;
  REQUIRE(sel_stride >= min_sel_stride(flags), "topk_filtering: sel_stride %u < %u", sel_stride,
          min_sel_stride(flags));
  // a score row is the candidate set; its length bounds the pages selected from
  const uint32_t max_row =
      aoakv::topk_max_pages() - ((flags & AOAKV_FLAG_QUEST_KERNEL) ? 1u : 0u);
  REQUIRE(score_stride >= 1u && score_stride <= max_row,
          "topk_filtering: score_stride %u not in [1, %u] (pages per row the top-k holds)",
          score_stride, max_row);
  aoakv::TopkArgs a{};
  a.scores = scores;
  a.score_stride = score_stride;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_last_page_len = kv_last_page_len;
  a.token_budget = token_budget;
  a.token_budgets = token_budgets;
  a.sel = sel_pages;
  a.sel_stride = sel_stride;
  a.Hkv = num_kv_heads;
  a.S = page_size;
  a.flags = flags;
  a.error = error_word;
  return hip_status(aoakv::launch_topk(a, batch_size, static_cast<hipStream_t>(stream)),
                    "topk_filtering");
}

size_t aoakv_decode_workspace_size(uint32_t batch_size, uint32_t num_qo_heads,
                                   uint32_t num_kv_heads, uint32_t head_dim,
                                   uint32_t max_sel_pages) {
  return ws_layout(batch_size, num_qo_heads, num_kv_heads, max_sel_pages, head_dim, nullptr,
                   nullptr);
}

// The one-launch layer's score handoff words follow the decode workspace's
// regions: B * Hkv * max_pages words, 256-byte aligned.
static size_t score_words_offset(size_t decode_bytes) { return round_up(decode_bytes, 256); }

size_t aoakv_layer_workspace_size(uint32_t batch_size, uint32_t num_qo_heads,
                                  uint32_t num_kv_heads, uint32_t head_dim,
                                  uint32_t max_sel_pages, uint32_t max_pages) {
  const size_t dec = ws_layout(batch_size, num_qo_heads, num_kv_heads, max_sel_pages, head_dim,
                               nullptr, nullptr);
  // score words: a copy per query head at most (self-selecting decode items
  // of GQA read one each)
  return score_words_offset(dec) + (size_t)batch_size * num_qo_heads * max_pages * 4u;
}

int aoakv_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  REQUIRE(workspace, "workspace_init: null workspace");
  REQUIRE(workspace_bytes % 4u == 0u, "workspace_init: size not a multiple of 4");
  return hip_status(aoakv::launch_fill_u32(static_cast<uint32_t*>(workspace),
                                           workspace_bytes / 4u, 0u,
                                           static_cast<hipStream_t>(stream)),
                    "workspace_init");
}

static int fill_decode(aoakv::DecodeArgs& a, Workspace& w, const void* q, void* o,
                       const void* kv_data, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* kv_last_page_len,
                       const int32_t* sel_pages, uint32_t sel_stride, uint32_t token_budget,
                       const int32_t* token_budgets, void* workspace, size_t workspace_bytes,
                       uint32_t batch_size, uint32_t max_pages, uint32_t num_qo_heads,
                       uint32_t num_kv_heads, uint32_t head_dim, uint32_t page_size,
                       uint32_t layout, uint32_t flags) {
  if (int e = check_shape(head_dim, page_size, layout, num_qo_heads)) return e;
  if (int e = check_group(num_qo_heads, num_kv_heads)) return e;
  REQUIRE(q && o && kv_data && kv_indptr && kv_indices && kv_last_page_len && workspace,
          "decode_sparse_attn: null pointer argument");
  REQUIRE(batch_size >= 1u && batch_size <= 65535u, "decode_sparse_attn: bad batch_size %u",
          batch_size);
  REQUIRE(max_pages >= 1u, "decode_sparse_attn: max_pages must be >= 1");
  const uint32_t max_sel = max_selected(sel_pages, sel_stride, token_budget, token_budgets,
                                        max_pages, page_size, flags);
  REQUIRE(!sel_pages || sel_stride >= min_sel_stride(flags), "decode_sparse_attn: sel_stride %u < %u",
          sel_stride, min_sel_stride(flags));
  // both decode kernels split each head's pages over chunks of 8 merged
  // through the workspace; the tuned merge holds at most decode_max_chunks
  // of them, the generic one (chunk order, one workgroup) any number
  const bool tuned = aoakv::tuned_shape(head_dim, page_size);
  REQUIRE(!tuned || aoakv::decode_chunks(max_sel) <= aoakv::decode_max_chunks(),
          "decode_sparse_attn: %u pages per head exceed the %u the split-K merge holds", max_sel,
          aoakv::decode_max_chunks() * 8u);
  const size_t need =
      ws_layout(batch_size, num_qo_heads, num_kv_heads, max_sel, head_dim, workspace, &w);
  REQUIRE(workspace_bytes >= need, "decode_sparse_attn: workspace of %zu bytes < %zu needed",
          workspace_bytes, need);
  a.q = static_cast<const aoakv::f16*>(q);
  a.o = static_cast<aoakv::f16*>(o);
  a.kv = static_cast<const aoakv::f16*>(kv_data);
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_last_page_len = kv_last_page_len;
  a.sel = sel_pages;
  a.sel_stride = sel_stride;
  a.token_budget = token_budget;
  a.token_budgets = token_budgets;
  a.partial = w.partial;
  a.counters = w.dec_counters;
  a.Hq = num_qo_heads;
  a.Hkv = num_kv_heads;
  a.S = page_size;
  a.max_chunks = aoakv::decode_chunks(max_sel);
  a.max_pages = max_pages;
  a.flags = flags & AOAKV_FLAG_QUEST_KERNEL;
  // grouped decode only where it changes anything (a group of 2 or more) and
  // the tuned kernels run (the generic ones serve one query head each)
  a.heads_per_item =
      (flags & AOAKV_FLAG_GROUPED_DECODE) && tuned ? num_qo_heads / num_kv_heads : 1u;
  a.g = aoakv::make_geom(layout, num_kv_heads, page_size, head_dim);
  a.error = w.ctl + aoakv::kErrWord;
  return AOAKV_OK;
}

int aoakv_decode_sparse_attn(const void* q, void* o, const void* kv_data,
                             const int32_t* kv_indptr, const int32_t* kv_indices,
                             const int32_t* kv_last_page_len, const int32_t* sel_pages,
                             uint32_t sel_stride, uint32_t token_budget,
                             const int32_t* token_budgets, void* workspace,
                             size_t workspace_bytes, uint32_t batch_size, uint32_t max_pages,
                             uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                             uint32_t page_size, uint32_t layout, uint32_t flags, void* stream) {
  if (int e = check_flags(flags, AOAKV_FLAG_QUEST_KERNEL | AOAKV_FLAG_GROUPED_DECODE,
                          "decode_sparse_attn"))
    return e;
  aoakv::DecodeArgs a{};
  Workspace w{};
  if (int e = fill_decode(a, w, q, o, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                          sel_pages, sel_stride, token_budget, token_budgets, workspace,
                          workspace_bytes, batch_size, max_pages, num_qo_heads, num_kv_heads,
                          head_dim, page_size, layout, flags))
    return e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(aoakv::tuned_shape(head_dim, page_size)
                        ? aoakv::launch_decode(a, batch_size, s)
                        : aoakv::launch_gen_decode(a, batch_size, head_dim, s),
                    "decode_sparse_attn");
}

int aoakv_sparse_decode_layer(const void* q, void* o, const void* kv_data,
                              const int32_t* kv_indptr, const int32_t* kv_indices,
                              const int32_t* kv_last_page_len, const void* metadata_data,
                              const int32_t* metadata_indptr, const int32_t* metadata_indices,
                              const void* v_log_norm, float* scores, uint32_t score_stride,
                              int32_t* sel_pages, uint32_t sel_stride, uint32_t token_budget,
                              const int32_t* token_budgets, void* workspace,
                              size_t workspace_bytes, uint32_t batch_size, uint32_t max_pages,
                              uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                              uint32_t page_size, uint32_t layout, uint32_t flags,
                              void* stream) {
  REQUIRE(sel_pages, "sparse_decode_layer: sel_pages is required");
  REQUIRE(max_pages <= aoakv::topk_max_pages(), "sparse_decode_layer: max_pages %u > %u",
          max_pages, aoakv::topk_max_pages());
  aoakv::EstimateArgs ea{};
  if (int e = fill_estimate(ea, q, scores, score_stride, metadata_data, metadata_indptr,
                            metadata_indices, kv_indptr, kv_indices, kv_last_page_len,
                            v_log_norm, batch_size, max_pages, num_qo_heads, num_kv_heads,
                            head_dim, page_size, layout, flags & ~AOAKV_FLAG_GROUPED_DECODE))
    return e;
  REQUIRE(sel_stride >= min_sel_stride(flags), "sparse_decode_layer: sel_stride %u < %u",
          sel_stride, min_sel_stride(flags));
  aoakv::DecodeArgs da{};
  Workspace w{};
  if (int e = fill_decode(da, w, q, o, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                          sel_pages, sel_stride, token_budget, token_budgets, workspace,
                          workspace_bytes, batch_size, max_pages, num_qo_heads, num_kv_heads,
                          head_dim, page_size, layout, flags))
    return e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  ea.flags &= kSelectFlags;
  ea.error = da.error;
  const bool tuned = aoakv::tuned_shape(head_dim, page_size);
  // the one-launch grid is one dimension of 256-thread workgroups (scoring
  // items, a top-k per kv head, decode items), and a dispatch counts its
  // work-items in 32 bits: a larger layer (1,024 sequences of 32 heads at
  // 512 decode chunks each, say) runs as the two launches, whose grids are
  // three-dimensional
  const uint64_t one_launch_grid =
      (uint64_t)batch_size * num_kv_heads *
          (aoakv::est_chunks(max_pages, num_qo_heads / num_kv_heads) + 1u) +
      (uint64_t)batch_size * (num_qo_heads / da.heads_per_item) * da.max_chunks;
  if (tuned && (flags & AOAKV_FLAG_SINGLE_LAUNCH) && max_pages <= aoakv::fused_topk_max_pages() &&
      one_launch_grid <= aoakv::layer_max_workgroups()) {
    // one launch: scoring, top-k and decode items of every head
    aoakv::LayerArgs la{};
    la.e = ea;
    la.e.sel = sel_pages;
    la.e.sel_stride = sel_stride;
    la.e.token_budget = token_budget;
    la.e.token_budgets = token_budgets;
    la.e.counters = w.est_counters;
    // handoff rows of the selection entries (the quest_kernel convention's
    // last page is not among them)
    const uint32_t sel_cap = max_selected(sel_pages, sel_stride, token_budget, token_budgets,
                                          max_pages, page_size, flags);
    const uint32_t max_sel = sel_cap < sel_stride ? sel_cap : sel_stride;
    la.e.hsel = w.hsel;
    la.e.hsel_stride = max_sel;
    la.e.hsel_gi = da.heads_per_item;
    la.d = da;
    la.d.hsel = w.hsel;
    la.d.hsel_stride = max_sel;
    la.d.hpart = w.hpart;
    // with room for them (aoakv_layer_workspace_size), the scores also go to
    // the top-k as handoff words, polled directly (no arrival counter)
    const size_t words_off = score_words_offset(w.bytes);
    const size_t words_row = (size_t)batch_size * num_kv_heads * max_pages * 4u;
    if (workspace_bytes >= words_off + words_row) {
      la.e.hscore = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + words_off);
      la.e.hscore_stride = max_pages;
      la.e.hscore_copies = 1u;
    }
    const uint32_t group = num_qo_heads / num_kv_heads;
    // self-selecting decode items read a copy of the score words per decode
    // block of the group, so each block's merging item clears its own
    const uint32_t copies = group / da.heads_per_item;
    // NHD: a head's metadata entries are 256-byte pieces 8 KB apart, so the
    // scoring items take two adjacent heads (512-byte runs) over half the
    // pages; they hand every score over as a word, so only with the words
    la.score_heads = layout == AOAKV_LAYOUT_NHD && group == 1u && num_kv_heads % 2u == 0u &&
                             la.e.hscore != nullptr
                         ? 2u
                         : 1u;
    la.est_chunks = aoakv::est_chunks(max_pages, group * la.score_heads);
    la.n_est = batch_size * (num_kv_heads / la.score_heads) * la.est_chunks;
    la.n_workers = aoakv::layer_score_workers(la.n_est, la.est_chunks);
    // (per scoring unit: est_chunks items of 128 / (group * score_heads)
    // pages over score_heads heads, the same bytes per item)
    la.stagger_ps = aoakv::layer_stagger_ps(la.est_chunks, group, batch_size * num_kv_heads);
    la.n_dec = batch_size * (num_qo_heads / da.heads_per_item) * da.max_chunks;
    // score words and the whole launch resident at once: each decode item
    // selects its kv head's pages itself (no top-k workgroups, no selection
    // handoff; with GQA every query head's items do, and the group's last
    // merging item clears the words).  With more workgroups than the GPU
    // holds, the 16 copies of every top-k cost more than the handoff they
    // save (config 5, 512 heads: 316 vs 250 us per layer).
    la.self_select = la.e.hscore != nullptr &&
                             workspace_bytes >= words_off + words_row * copies &&
                             la.n_workers + la.n_dec <=
                                 resident_layer_workgroups(num_qo_heads / num_kv_heads,
                                                           da.heads_per_item, la.score_heads)
                         ? 1u
                         : 0u;
    la.n_heads = la.self_select ? 0u : batch_size * num_kv_heads;
    if (la.self_select) la.e.hscore_copies = copies;
    return hip_status(aoakv::launch_layer(la, s), "sparse_decode_layer");
  }
  if (tuned && max_pages <= aoakv::fused_topk_max_pages()) {
    // two launches: the scores alone (the unfused kernel, smaller items),
    // then decode items that each select their kv head's pages from the
    // complete scores (16 copies of every top-k, none waiting on another
    // workgroup) and write their chunk's entries of sel_pages.  Config 2:
    // 23.0 us per layer (7.9 + 15.1), against 24.1 with the top-k fused into
    // the scoring launch's last item per head (13.0 + 11.1); before the
    // streamed loads 24.7-25.1 against 25.6, and starting the kv heads'
    // decode items 0.1-0.3 us apart was slower (25.1-30.0).
    if (int e = hip_status(aoakv::launch_estimate(ea, batch_size, max_pages, s), "estimate"))
      return e;
    aoakv::EstimateArgs es = ea;
    es.sel = sel_pages;
    es.sel_stride = sel_stride;
    es.token_budget = token_budget;
    es.token_budgets = token_budgets;
    return hip_status(aoakv::launch_decode(da, batch_size, s, &es), "sparse_decode_layer/decode");
  }
  if (int e = launch_estimate_topk(ea, w, sel_pages, sel_stride, token_budget, token_budgets,
                                   batch_size, max_pages, head_dim, page_size, flags, s))
    return e;
  return hip_status(tuned ? aoakv::launch_decode(da, batch_size, s)
                          : aoakv::launch_gen_decode(da, batch_size, head_dim, s),
                    "sparse_decode_layer/decode");
}

int aoakv_sparse_decode_layer_noalloc(
    const void* q, void* o, const void* kv_data, const int32_t* kv_indptr,
    const int32_t* kv_indices, const int32_t* kv_last_page_len, const void* metadata_data,
    const int32_t* metadata_indptr, const int32_t* metadata_indices, const void* v_log_norm,
    float* scores, uint32_t score_stride, int32_t* sel_pages, uint32_t sel_stride,
    uint32_t token_budget, const int32_t* token_budgets, uint32_t batch_size, uint32_t max_pages,
    uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim, uint32_t page_size,
    uint32_t layout, uint32_t flags, void* stream) {
  REQUIRE(!(flags & AOAKV_FLAG_SINGLE_LAUNCH),
          "sparse_decode_layer_noalloc: runs the two-launch path only (AOAKV_FLAG_SINGLE_LAUNCH "
          "needs a workspace the caller can re-initialise after a wait gave up)");
  // the decode workspace this call lays out must fit the scratch array
  const uint32_t max_sel = max_selected(sel_pages, sel_stride, token_budget, token_budgets,
                                        max_pages, page_size, flags);
  const size_t need =
      ws_layout(batch_size, num_qo_heads, num_kv_heads, max_sel, head_dim, nullptr, nullptr);
  REQUIRE(need <= kNoAllocScratchBytes,
          "sparse_decode_layer_noalloc: this call needs %zu bytes of scratch, more than the "
          "%zu the library holds per device (batch %u x %u query heads x %u selected pages)",
          need, kNoAllocScratchBytes, batch_size, num_qo_heads, max_sel);
  void* ws = nullptr;
  if (int e = scratch_for_current_device(&ws, "sparse_decode_layer_noalloc")) return e;
  return aoakv_sparse_decode_layer(q, o, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                                   metadata_data, metadata_indptr, metadata_indices, v_log_norm,
                                   scores, score_stride, sel_pages, sel_stride, token_budget,
                                   token_budgets, ws, kNoAllocScratchBytes, batch_size, max_pages,
                                   num_qo_heads, num_kv_heads, head_dim, page_size, layout, flags,
                                   stream);
}

int aoakv_noalloc_init(void) {
  void* ws = nullptr;
  return scratch_for_current_device(&ws, "noalloc_init");
}

int aoakv_noalloc_error(uint32_t* error_bits, uint32_t clear, void* stream) {
  REQUIRE(error_bits, "noalloc_error: null error_bits");
  void* ws = nullptr;
  if (int e = scratch_for_current_device(&ws, "noalloc_error")) return e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* word = static_cast<uint32_t*>(ws) + aoakv::kErrWord;
  // the word as the stream's earlier calls leave it; a synchronous copy to a
  // stack word (no staging buffer of the library's own)
  if (hipError_t e = hipStreamSynchronize(s); e != hipSuccess)
    return fail(AOAKV_ERR_HIP, "noalloc_error: hipStreamSynchronize: %s", hipGetErrorString(e));
  uint32_t bits = 0u;
  if (hipError_t e = hipMemcpy(&bits, word, sizeof bits, hipMemcpyDeviceToHost); e != hipSuccess)
    return fail(AOAKV_ERR_HIP, "noalloc_error: hipMemcpy: %s", hipGetErrorString(e));
  *error_bits = bits;
  if (clear && bits != 0u) {
    if (hipError_t e = aoakv::launch_fill_u32(word, 1u, 0u, s); e != hipSuccess)
      return fail(AOAKV_ERR_HIP, "noalloc_error: clear: %s", hipGetErrorString(e));
  }
  return AOAKV_OK;
}

int aoakv_estimate_topk(const void* q, const void* metadata_data, const int32_t* metadata_indptr,
                        const int32_t* metadata_indices, const int32_t* kv_indptr,
                        const int32_t* kv_indices, const int32_t* kv_last_page_len,
                        const void* v_log_norm, float* scores, uint32_t score_stride,
                        int32_t* sel_pages, uint32_t sel_stride, uint32_t token_budget,
                        const int32_t* token_budgets, void* workspace, size_t workspace_bytes,
                        uint32_t batch_size, uint32_t max_pages, uint32_t num_qo_heads,
                        uint32_t num_kv_heads, uint32_t head_dim, uint32_t page_size,
                        uint32_t layout, uint32_t flags, void* stream) {
  REQUIRE(sel_pages && workspace, "estimate_topk: sel_pages and workspace are required");
  REQUIRE(max_pages <= aoakv::topk_max_pages(), "estimate_topk: max_pages %u > %u", max_pages,
          aoakv::topk_max_pages());
  REQUIRE(sel_stride >= min_sel_stride(flags), "estimate_topk: sel_stride %u < %u", sel_stride,
          min_sel_stride(flags));
  aoakv::EstimateArgs ea{};
  if (int e = fill_estimate(ea, q, scores, score_stride, metadata_data, metadata_indptr,
                            metadata_indices, kv_indptr, kv_indices, kv_last_page_len,
                            v_log_norm, batch_size, max_pages, num_qo_heads, num_kv_heads,
                            head_dim, page_size, layout, flags))
    return e;
  Workspace w{};
  const uint32_t max_sel = sel_stride < max_pages ? sel_stride : max_pages;
  const size_t need =
      ws_layout(batch_size, num_qo_heads, num_kv_heads, max_sel, head_dim, workspace, &w);
  REQUIRE(workspace_bytes >= need, "estimate_topk: workspace of %zu bytes < %zu needed",
          workspace_bytes, need);
  ea.error = w.ctl + aoakv::kErrWord;
  return launch_estimate_topk(ea, w, sel_pages, sel_stride, token_budget, token_budgets,
                              batch_size, max_pages, head_dim, page_size, flags,
                              static_cast<hipStream_t>(stream));
}

int aoakv_prefill_with_paged_kv_cache(const void* q, void* o, const void* kv_data,
                                      const int32_t* kv_indices, uint32_t num_kv_pages,
                                      uint32_t kv_last_page_len, uint32_t qo_len,
                                      uint32_t causal, uint32_t num_qo_heads,
                                      uint32_t num_kv_heads, uint32_t head_dim,
                                      uint32_t page_size, uint32_t layout, void* stream) {
  if (int e = check_shape(head_dim, page_size, layout, num_qo_heads)) return e;
  if (num_kv_heads == 0u || num_qo_heads % num_kv_heads != 0u)
    return fail(AOAKV_ERR_INVALID,
                "prefill_with_paged_kv_cache: num_qo_heads %u not a multiple of num_kv_heads %u",
                num_qo_heads, num_kv_heads);
  REQUIRE(q && o && kv_data && kv_indices, "prefill_with_paged_kv_cache: null pointer argument");
  REQUIRE(num_kv_pages >= 1u, "prefill_with_paged_kv_cache: num_kv_pages must be >= 1");
  REQUIRE(kv_last_page_len >= 1u && kv_last_page_len <= page_size,
          "prefill_with_paged_kv_cache: kv_last_page_len %u not in [1, %u]", kv_last_page_len,
          page_size);
  const uint64_t L = (uint64_t)(num_kv_pages - 1u) * page_size + kv_last_page_len;
  REQUIRE(qo_len >= 1u && qo_len <= L,
          "prefill_with_paged_kv_cache: qo_len %u not in [1, %llu]", qo_len,
          (unsigned long long)L);
  REQUIRE(L < (1ull << 31), "prefill_with_paged_kv_cache: sequence too long");
  aoakv::PrefillArgs a{};
  a.q = static_cast<const aoakv::f16*>(q);
  a.o = static_cast<aoakv::f16*>(o);
  a.kv = static_cast<const aoakv::f16*>(kv_data);
  a.kv_indices = kv_indices;
  a.H = num_kv_heads;
  a.Hq = num_qo_heads;
  a.L = (uint32_t)L;
  a.Lq = qo_len;
  a.causal = causal ? 1u : 0u;
  a.sm_scale = 1.0f / std::sqrt((float)head_dim);
  a.g = aoakv::make_geom(layout, num_kv_heads, page_size, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(aoakv::prefill_tuned_shape(head_dim, page_size)
                        ? aoakv::launch_prefill(a, page_size, head_dim, s)
                        : aoakv::launch_gen_prefill(a, head_dim, s),
                    "prefill_with_paged_kv_cache");
}

}  // extern "C"
