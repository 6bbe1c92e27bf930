// Kernels for the shapes the tuned kernels do not take (gfx950): head_dim
// 64, 128 or 256 with any page size 1..32, except (128, 16), which has the
// tuned kernels of append.hip, decode.hip and prefill.hip.  The reference
// instantiates its kernels per head_dim (SWITCH_HEAD_DIM, decode_page.cuh:
// 718-760, decode_attn.cuh:1159) and per prefill page size (prefill.cuh:
// 1032-1036); here the other shapes share one simpler set of kernels with
// the same semantics and argument blocks:
//   * a D-dim fp16 vector is held by D/8 consecutive lanes, 8 dims per lane
//     (a "lane group": 8 lanes for D = 64, 16 for 128, 32 for 256), and
//     reductions inside a group are butterflies of wave shuffles;
//   * page scores: one lane group per page, then the existing top-k kernel
//     (which takes any page size);
//   * decode: split over chunks of kGenChunkPages selected pages, one
//     workgroup per (chunk, query head, sequence), online softmax per lane
//     group, merged in LDS, then across chunks by the last to arrive;
//   * prefill: one lane group per query, keys in order with an online
//     softmax, no MFMA (the tuned MFMA kernel covers (128, 16)).
// Arithmetic follows the tuned kernels where they define the reference's
// rounding (fp16 filters, the fp32 page mean with one rounding, the fp16
// running mean, the sequential fp32 norm of the log-norm, fp16 logits
// rounded before and after the 1/sqrt(d) division).
#include "kernels.hpp"

namespace aoakv {
namespace {

// sum / max over the N lanes of this lane's group (N a power of two <= 32);
// every lane of the group gets the result
template <uint32_t N>
__device__ inline float grp_sum(float x) {
#pragma unroll
  for (uint32_t m = 1; m < N; m <<= 1) x += __shfl_xor(x, (int)m, kWave);
  return x;
}

// The same sum over a lane group through DPP within a row (and, for 32
// lanes, one LDS permute between the two rows) instead of LDS permutes
// throughout: a few cycles per DPP step where a permute waits on the LDS
// unit.  Groups are aligned to half-rows (N = 8), rows (16) or row pairs
// (32), so every lane read belongs to the same group.  (Another summation
// order than grp_sum.)
template <uint32_t N>
__device__ inline float grp_sum_dpp(float x) {
  static_assert(N == 8u || N == 16u || N == 32u, "lane groups of 8, 16 or 32");
  x = x + dpp<kQuadSwap1>(x);
  x = x + dpp<kQuadSwap2>(x);
  x = x + dpp<kRowHalfMirror>(x);
  if constexpr (N >= 16u) x = x + dpp<kRowMirror>(x);
  if constexpr (N == 32u) x = x + __shfl_xor(x, 16, kWave);
  return x;
}

// sqrt(D) as the fp32 the simulation divides by (math.sqrt(head_dim))
template <int D>
__device__ __host__ constexpr float sqrt_d() {
  return D == 64 ? 8.0f : D == 256 ? 16.0f : kSqrtHeadDim;
}

// log(norm(V̄) + 1e-8) of one D-dim fp16 vector held by an N-lane group, as
// log_norm_row: fp32 sum of squares in dim order, carried lane to lane,
// correctly rounded root, fp16 rounding after each op.
template <uint32_t N>
__device__ inline f16 grp_log_norm(const H8& vbar, uint32_t l) {
  const uint32_t base = __lane_id() & ~(N - 1u);
  float acc = 0.f;
#pragma unroll
  for (uint32_t src = 0; src < N; ++src) {
    if (l == src) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float x = (float)vbar.v[j];
        const float sq = x * x;
        acc = acc + sq;
      }
    }
    acc = __shfl(acc, (int)(base | src), kWave);
  }
  f16 nrm = r16((float)__builtin_sqrt((double)acc));
  nrm = r16((float)nrm + 1e-8f);
  return r16((float)log((double)(float)nrm));
}

// RoPE of the 8 dims lane l of an N-lane group holds (D = 8N dims), at
// position pos: rotate-half with the partner dims d +- D/2 in lane l ^ N/2.
template <uint32_t N>
__device__ inline H8 grp_rope(const H8& x, uint32_t pos, uint32_t l, const float* freqs) {
  constexpr uint32_t D = 8u * N;
  const uint4 u = __builtin_bit_cast(uint4, x);
  uint4 pu;
  pu.x = (uint32_t)__shfl_xor((int)u.x, (int)(N / 2u), kWave);
  pu.y = (uint32_t)__shfl_xor((int)u.y, (int)(N / 2u), kWave);
  pu.z = (uint32_t)__shfl_xor((int)u.z, (int)(N / 2u), kWave);
  pu.w = (uint32_t)__shfl_xor((int)u.w, (int)(N / 2u), kWave);
  const H8 p = __builtin_bit_cast(H8, pu);
  const bool low = l < N / 2u;
  H8 y;
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const uint32_t i = (l * kVec + (uint32_t)j) % (D / 2u);
    float s, c;
    sincosf((float)pos * freqs[i], &s, &c);
    const float a = (float)x.v[j] * c;
    const float b = (float)p.v[j] * s;
    y.v[j] = r16(low ? a - b : a + b);
  }
  return y;
}

// ---------------------------------------------------------------- append
// One lane group per (page, head) as append_prefill_kernel; 256 / (D/8)
// heads per workgroup.
template <int D>
__global__ __launch_bounds__(256) void gen_append_prefill_kernel(AppendPrefillArgs a) {
  constexpr uint32_t N = D / 8, HPB = 256u / N;
  const uint32_t l = threadIdx.x % N;
  const uint32_t h = blockIdx.y * HPB + threadIdx.x / N;
  const uint32_t p = a.first_page + blockIdx.x;
  if (h >= a.H || p >= a.num_pages) return;  // whole groups exit together

  const uint32_t S = a.S;
  const uint32_t L = (a.num_pages - 1u) * S + a.last_page_len;
  const uint32_t start = L - a.N;
  const uint32_t e0 = start > p * S ? start - p * S : 0u;
  const uint32_t e1 = (L - p * S) < S ? (L - p * S) : S;
  const uint32_t phys = (uint32_t)a.kv_indices[p];
  const uint32_t mpage = (uint32_t)a.meta_indices[p / S];
  const uint32_t ment = p % S;
  const uint32_t d0 = l * kVec;

  f16* kmax_p = a.meta + elem_off(a.g, mpage, 0, h, ment) + d0;
  f16* kmin_p = a.meta + elem_off(a.g, mpage, 1, h, ment) + d0;
  f16* vbar_p = a.v_mean + ((size_t)phys * a.H + h) * D + d0;
  H8 kmax, kmin, vbar;
  float vsum[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) vsum[j] = 0.f;
  if (e0 > 0u) {
    kmax = ld16(kmax_p);
    kmin = ld16(kmin_p);
    vbar = ld16(vbar_p);
  } else {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      kmax.v[j] = (f16)-65504.0f;
      kmin.v[j] = (f16)65504.0f;
    }
  }
  const size_t in_row = (size_t)a.H * D;
  const f16* kin = a.k + (size_t)(p * S + e0 - start) * in_row + (size_t)h * D + d0;
  const f16* vin = a.v + (size_t)(p * S + e0 - start) * in_row + (size_t)h * D + d0;
  f16* kout = a.kv + elem_off(a.g, phys, 0, h, e0) + d0;
  f16* vout = a.kv + elem_off(a.g, phys, 1, h, e0) + d0;
  const uint32_t n = e1 - e0;
  for (uint32_t i = 0; i < n; ++i) {
    const H8 kk = ld16(kin + i * in_row);
    const H8 vv = ld16(vin + i * in_row);
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      kmax.v[j] = kk.v[j] > kmax.v[j] ? kk.v[j] : kmax.v[j];
      kmin.v[j] = kk.v[j] < kmin.v[j] ? kk.v[j] : kmin.v[j];
      if (e0 == 0u) vsum[j] = vsum[j] + (float)vv.v[j];       // page filled from empty
      else vbar.v[j] = running_mean(vbar.v[j], vv.v[j], e0 + i);  // tokens added to a page
    }
    st16(kout + (size_t)i * a.g.tok, kk);
    st16(vout + (size_t)i * a.g.tok, vv);
  }
  if (e0 == 0u) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) vbar.v[j] = r16(vsum[j] / (float)n);
  }
  st16(kmax_p, kmax);
  st16(kmin_p, kmin);
  st16(vbar_p, vbar);
  const f16 lvn = grp_log_norm<N>(vbar, l);
  if (l == 0u) a.v_log_norm[(size_t)phys * a.H + h] = lvn;
}

// One new token per sequence, as append_decode_kernel (with ROPE: the block
// rows past the kv heads rotate q in place and k is rotated before the
// append).
template <int D, bool ROPE>
__global__ __launch_bounds__(256) void gen_append_decode_kernel(AppendDecodeArgs a) {
  constexpr uint32_t N = D / 8, HPB = 256u / N;
  const uint32_t l = threadIdx.x % N;
  const uint32_t b = blockIdx.x;
  const uint32_t kv_blocks = (a.H + HPB - 1) / HPB;
  const bool q_block = ROPE && blockIdx.y >= kv_blocks;
  const uint32_t h = (q_block ? blockIdx.y - kv_blocks : blockIdx.y) * HPB + threadIdx.x / N;
  if (h >= (q_block ? a.Hq : a.H)) return;

  const uint32_t S = a.S;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  const uint32_t lpl = (uint32_t)a.kv_last_page_len[b];
  if (P == 0u || lpl == 0u || lpl > S) return;
  const uint32_t pos = (P - 1u) * S + lpl - 1u;
  if constexpr (ROPE) {
    if (q_block) {
      f16* qp = a.q + ((size_t)b * a.Hq + h) * D + l * kVec;
      st16(qp, grp_rope<N>(ld16(qp), pos, l, a.rope_f.f));
      return;
    }
  }
  const uint32_t e = lpl - 1u;
  const uint32_t p = P - 1u;
  const uint32_t phys = (uint32_t)a.kv_indices[pbeg + p];
  const uint32_t mpage = (uint32_t)a.meta_indices[(uint32_t)a.meta_indptr[b] + p / S];
  const uint32_t ment = p % S;
  const uint32_t d0 = l * kVec;
  f16* kmax_p = a.meta + elem_off(a.g, mpage, 0, h, ment) + d0;
  f16* kmin_p = a.meta + elem_off(a.g, mpage, 1, h, ment) + d0;
  f16* vbar_p = a.v_mean + ((size_t)phys * a.H + h) * D + d0;
  const size_t in_off = ((size_t)b * a.H + h) * D + d0;
  H8 kk = ld16(a.k + in_off);
  const H8 vv = ld16(a.v + in_off);
  if constexpr (ROPE) {
    kk = grp_rope<N>(kk, pos, l, a.rope_f.f);
    st16(a.k + in_off, kk);
  }
  H8 kmax, kmin, vbar;
  if (e == 0u) {
    kmax = kk;
    kmin = kk;
    vbar = vv;
  } else {
    kmax = ld16(kmax_p);
    kmin = ld16(kmin_p);
    vbar = ld16(vbar_p);
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      kmax.v[j] = kk.v[j] > kmax.v[j] ? kk.v[j] : kmax.v[j];
      kmin.v[j] = kk.v[j] < kmin.v[j] ? kk.v[j] : kmin.v[j];
      vbar.v[j] = running_mean(vbar.v[j], vv.v[j], e);
    }
  }
  st16(a.kv + elem_off(a.g, phys, 0, h, e) + d0, kk);
  st16(a.kv + elem_off(a.g, phys, 1, h, e) + d0, vv);
  st16(kmax_p, kmax);
  st16(kmin_p, kmin);
  st16(vbar_p, vbar);
  const f16 lvn = grp_log_norm<N>(vbar, l);
  if (l == 0u) a.v_log_norm[(size_t)phys * a.H + h] = lvn;
}

// In-place RoPE of q [n, Hq, D] and k [n, Hkv, D] at positions past + n.
template <int D>
__global__ __launch_bounds__(256) void gen_rope_kernel(RopeArgs a) {
  constexpr uint32_t N = D / 8, HPB = 256u / N;
  const uint32_t l = threadIdx.x % N;
  const uint32_t n = blockIdx.x;
  for (uint32_t h = threadIdx.x / N; h < a.Hq + a.Hkv; h += HPB) {
    f16* p = h < a.Hq ? a.q + ((size_t)n * a.Hq + h) * D
                      : a.k + ((size_t)n * a.Hkv + (h - a.Hq)) * D;
    p += l * kVec;
    st16(p, grp_rope<N>(ld16(p), a.past + n, l, a.rope_f.f));
  }
}

// ---------------------------------------------------------------- page scores
// Pages [64 x, 64 x + 64) of (sequence b, kv head h): one lane group per
// page.  Score of a page (filter_util.py:269-330, as score_item): per query
// head g of the group, x_g = sum_d max(q_d Kmax_d, q_d Kmin_d) (fp32); the
// value-aware score is logsumexp_g(2 x_g / sqrt(d)) + 2 log-norm, plain
// Quest sums x_g over the group.
constexpr uint32_t kGenPagesPerBlock = 64;

template <int D, int GROUP>
__global__ __launch_bounds__(256) void gen_estimate_kernel(EstimateArgs a) {
  constexpr uint32_t N = D / 8, PPS = 256u / N;  // pages per step of the block
  const uint32_t l = threadIdx.x % N;
  const uint32_t b = blockIdx.z, h = blockIdx.y;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P0 = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  const bool quest = (a.flags & kFlagQuestKernel) != 0u;
  uint32_t P = P0;
  const uint32_t rowcap = a.score_stride + (quest ? 1u : 0u);
  if (P > rowcap) P = rowcap;
  if (P > a.max_pages) P = a.max_pages;
  if (P != P0 && blockIdx.x == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  const uint32_t nstore = quest ? (P == 0u ? 0u : P - 1u) : P;
  const uint32_t mbeg = (uint32_t)a.meta_indptr[b];
  const bool value_aware = (a.flags & kFlagValueAware) != 0u;
  H8 q[GROUP];
#pragma unroll
  for (int g = 0; g < GROUP; ++g)
    q[g] = ld16(a.q + ((size_t)b * a.Hq + h * GROUP + g) * D + l * kVec);
  const uint32_t pb = blockIdx.x * kGenPagesPerBlock;  // the block's first page
  if (pb >= nstore) return;                            // uniform
  const uint32_t p_end = pb + kGenPagesPerBlock < nstore ? pb + kGenPagesPerBlock : nstore;
  // The block's pages in kSt steps of PPS, group g taking page pb + g + s *
  // PPS at step s.  Every step's page-table words are loaded together, then
  // every step's metadata and value statistic (unconditional loads of
  // clamped pages: a page past the block's end reads its first), so the
  // block waits on two round trips, not two or three per step; the scores
  // are computed in the same order as step by step.
  constexpr uint32_t kSt = kGenPagesPerBlock / PPS;
  uint32_t mpg[kSt], phys[kSt];
#pragma unroll
  for (uint32_t st = 0; st < kSt; ++st) {
    const uint32_t p = pb + threadIdx.x / N + st * PPS;
    const uint32_t pc = p < p_end ? p : pb;
    mpg[st] = (uint32_t)a.meta_indices[mbeg + pc / a.S];
    phys[st] = value_aware ? (uint32_t)a.kv_indices[pbeg + pc] : 0u;
  }
  H8 kmxs[kSt], kmns[kSt];
  f16 lvn[kSt];
#pragma unroll
  for (uint32_t st = 0; st < kSt; ++st) {
    const uint32_t p = pb + threadIdx.x / N + st * PPS;
    const uint32_t pc = p < p_end ? p : pb;
    const size_t off = elem_off(a.g, mpg[st], 0, h, pc % a.S) + l * kVec;
    // read once: non-temporal loads, as the tuned scoring's
    kmxs[st] = ld16_nt(a.meta + off);
    kmns[st] = ld16_nt(a.meta + off + a.g.kv);
    lvn[st] = value_aware ? a.v_log_norm[(size_t)phys[st] * a.Hkv + h] : (f16)0.f;
  }
#pragma unroll
  for (uint32_t st = 0; st < kSt; ++st) {
    const uint32_t p = pb + threadIdx.x / N + st * PPS;
    if (p >= p_end) break;  // (whole lane groups; later steps lie further on)
    const H8 kmx = kmxs[st], kmn = kmns[st];
    float x[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float qv = (float)q[g].v[j];
        acc = acc + fmaxf(qv * (float)kmx.v[j], qv * (float)kmn.v[j]);
      }
      x[g] = grp_sum_dpp<N>(acc);
    }
    float score;
    if (value_aware) {
      float m = -INFINITY;
#pragma unroll
      for (int g = 0; g < GROUP; ++g) {
        x[g] = 2.0f * (x[g] / sqrt_d<D>());
        m = fmaxf(m, x[g]);
      }
      score = x[0];
      if (GROUP > 1) {
        float se = 0.f;
#pragma unroll
        for (int g = 0; g < GROUP; ++g) se = se + expf(x[g] - m);
        score = logf(se) + m;
      }
      score = score + 2.0f * (float)lvn[st];
    } else {
      score = x[0];
#pragma unroll
      for (int g = 1; g < GROUP; ++g) score = score + x[g];
    }
    if (l == 0u) a.scores[((size_t)b * a.Hkv + h) * a.score_stride + p] = score;
  }
}

// ---------------------------------------------------------------- decode
// Attention of query head hq of sequence b over its selected pages (or all
// of them), split over chunks of kGenChunkPages entries: one workgroup per
// (chunk, query head, sequence) of W waves; wave w takes the chunk's entries
// w, w + W, ..., lane group v of a wave the page's tokens v, v + 64/N, ...
// W = 8 (a page per wave) when the grid has no more workgroups than the GPU
// has CUs, else 4 (fewer registers per workgroup, more of them resident).
// Logits fp16(q.k), then fp16(. / sqrt(d)) (quest_attention.py:265-268); online
// softmax in fp32; the groups' (m, l, o) merged in LDS into the chunk's
// partial.  A head of one chunk writes its output directly; otherwise the
// last chunk to arrive at the head's counter merges the partials in chunk
// order (the same arithmetic whichever workgroup merges) and clears them.
// The quest_kernel convention attends the last page after the nsel selected
// ones.
// STREAM: no GQA group shares the pages' K/V, which are then loaded
// non-temporally (as in the tuned decode)
template <int D, uint32_t W, bool STREAM>
__global__ __launch_bounds__(W * 64) void gen_decode_kernel(DecodeArgs a) {
  static_assert(W == 4u || W == 8u, "4 or 8 waves");
  constexpr uint32_t N = D / 8, GPW = kWave / N, G = W * GPW;  // groups per wave / block
  constexpr uint32_t kStride = (uint32_t)D + 4u;                // partial: o[D], m, l, pad
  __shared__ float s_o[G][D];
  __shared__ float s_ml[G][2];
  __shared__ uint32_t s_last;
  const uint32_t l = threadIdx.x % N, grp = threadIdx.x / N;
  const uint32_t wave = threadIdx.x / kWave, v = grp % GPW;
  const uint32_t chunk = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
  const uint32_t hkv = hq / (a.Hq / a.Hkv);
  const bool quest = (a.flags & kFlagQuestKernel) != 0u;
  const uint32_t S = a.S;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P_table = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  const uint32_t P = P_table < a.max_pages ? P_table : a.max_pages;
  if (P != P_table && chunk == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  const uint32_t lpl = (uint32_t)a.kv_last_page_len[b];
  if (P == 0u || lpl == 0u || lpl > S) return;  // malformed page table
  const uint32_t budget = a.token_budgets ? (uint32_t)a.token_budgets[b] : a.token_budget;
  uint32_t npages = P;
  if (a.sel != nullptr) {
    npages = num_selected_pages((P - 1u) * S + lpl, budget, S, P, quest ? kFlagQuestKernel : 0u);
    const uint32_t row_cap = a.sel_stride + (quest ? 1u : 0u);
    if (npages > row_cap) npages = row_cap;
  }
  // the grid holds max_chunks chunks per head: never index partials past it
  if (npages > a.max_chunks * kGenChunkPages) {
    npages = a.max_chunks * kGenChunkPages;
    if (chunk == 0u && threadIdx.x == 0u) flag_error(a.error, kErrTruncated);
  }
  const uint32_t nch = (npages + kGenChunkPages - 1u) / kGenChunkPages;
  if (chunk >= nch) return;  // uniform per block
  const uint32_t nsel = (quest && a.sel != nullptr) ? npages - 1u : npages;
  const int32_t* sel_row = a.sel ? a.sel + ((size_t)b * a.Hkv + hkv) * a.sel_stride : nullptr;
  const uint32_t last_phys = (uint32_t)a.kv_indices[pbeg + P - 1u];
  const H8 q = ld16(a.q + ((size_t)b * a.Hq + hq) * D + l * kVec);

  float m = -INFINITY, lsum = 0.f, o[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) o[j] = 0.f;
  const uint32_t ib = chunk * kGenChunkPages;  // the chunk's first entry (< npages)
  const uint32_t i1 = ib + kGenChunkPages < npages ? ib + kGenChunkPages : npages;
  // The wave's pages, entries ib + wave, ib + wave + W, ..., and their token
  // counts (0: no page).  Group v takes tokens v, v + GPW, ... of each.  The
  // K/V loads go out in batches of kB (page, token) slots, all of a batch
  // before any is used (unconditional loads of clamped addresses: a slot
  // past its page's tokens reads the page's slot 0, a missing page the
  // chunk's first), so a wave waits on memory once per batch instead of
  // once per token slot; the arithmetic runs in the same order as token by
  // token.
  constexpr uint32_t kPPW = kGenChunkPages / W;              // pages per wave
  constexpr uint32_t kTPG = (kMaxPageSize + GPW - 1u) / GPW;  // token slots of a group per page
  constexpr uint32_t kF = kPPW * kTPG;                        // ... over the wave's pages
  constexpr uint32_t kB = kF < 8u ? kF : 8u;                  // slots loaded together
  uint32_t ph[kPPW], nt[kPPW];
#pragma unroll
  for (uint32_t k = 0; k < kPPW; ++k) {
    const uint32_t i = ib + wave + W * k;
    const uint32_t ic = i < i1 ? i : ib;
    uint32_t phys;
    if (a.sel == nullptr) phys = (uint32_t)a.kv_indices[pbeg + ic];
    else phys = ic < nsel ? (uint32_t)sel_row[ic] : last_phys;
    ph[k] = phys;
    nt[k] = i < i1 ? (phys == last_phys ? lpl : S) : 0u;
  }
  for (uint32_t f0 = 0; f0 < kF; f0 += kB) {
    H8 kk[kB], vv[kB];
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) {
      const uint32_t f = f0 + u, k = f / kTPG, j = f % kTPG;
      if (GPW * j >= S) continue;  // uniform: slots past the page size
      const uint32_t t = v + GPW * j;
      const uint32_t tc = t < nt[k] ? t : 0u;
      const f16* kp = a.kv + elem_off(a.g, ph[k], 0, hkv, tc) + l * kVec;
      const f16* vp = a.kv + elem_off(a.g, ph[k], 1, hkv, tc) + l * kVec;
      kk[u] = STREAM ? ld16_nt(kp) : ld16(kp);
      vv[u] = STREAM ? ld16_nt(vp) : ld16(vp);
    }
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) {
      const uint32_t f = f0 + u, k = f / kTPG, j = f % kTPG;
      const uint32_t t = v + GPW * j;
      if (GPW * j >= S || t >= nt[k]) continue;  // (whole lane groups)
      float acc = 0.f;
#pragma unroll
      for (int jj = 0; jj < kVec; ++jj) acc = acc + (float)q.v[jj] * (float)kk[u].v[jj];
      const float x = (float)r16((float)r16(grp_sum_dpp<N>(acc)) / sqrt_d<D>());
      const float mn = fmaxf(m, x);
      const float c = m == -INFINITY ? 0.f : __expf(m - mn);
      const float p = __expf(x - mn);
      lsum = lsum * c + p;
#pragma unroll
      for (int jj = 0; jj < kVec; ++jj) o[jj] = o[jj] * c + p * (float)vv[u].v[jj];
      m = mn;
    }
  }
#pragma unroll
  for (int j = 0; j < kVec; ++j) s_o[grp][l * kVec + j] = o[j];
  if (l == 0u) {
    s_ml[grp][0] = m;
    s_ml[grp][1] = lsum;
  }
  __syncthreads();
  const size_t bh = (size_t)b * a.Hq + hq;
  const uint32_t d = threadIdx.x;
  if (d < (uint32_t)D) {
    float M = -INFINITY;
    for (uint32_t g2 = 0; g2 < G; ++g2) M = fmaxf(M, s_ml[g2][0]);
    float acc = 0.f, Ls = 0.f;
    for (uint32_t g2 = 0; g2 < G; ++g2) {
      const float w = s_ml[g2][0] == -INFINITY ? 0.f : __expf(s_ml[g2][0] - M);
      acc = acc + w * s_o[g2][d];
      Ls = Ls + w * s_ml[g2][1];
    }
    if (nch == 1u) {
      a.o[bh * D + d] = r16(acc / Ls);
    } else {
      float* part = a.partial + (bh * a.max_chunks + chunk) * kStride;
      st_agent(part + d, acc);
      if (d == 0u) {
        st_agent(part + D, M);
        st_agent(part + D + 1u, Ls);
      }
    }
  }
  if (nch == 1u) return;
  if (!arrive_last(&a.counters[bh * kCounterStride], nch, &s_last)) return;
  // the last chunk to arrive: merge every chunk's partial in chunk order,
  // then clear the partials (the whole workspace stays zero between calls)
  if (d < (uint32_t)D) {
    // in groups of 16 chunks, every load of a group issued before any is
    // used (one memory round trip per group), folded in chunk order
    const float* base = a.partial + bh * a.max_chunks * kStride;
    float M = -INFINITY, Ls = 0.f, acc = 0.f;
    for (uint32_t c0 = 0; c0 < nch; c0 += 16u) {
      float mc[16], lc[16], oc[16];
#pragma unroll
      for (uint32_t u = 0; u < 16u; ++u) {
        const float* part = base + (c0 + u < nch ? c0 + u : nch - 1u) * kStride;
        mc[u] = ld_agent(part + D);
        lc[u] = ld_agent(part + D + 1u);
        oc[u] = ld_agent(part + d);
      }
#pragma unroll
      for (uint32_t u = 0; u < 16u; ++u) {
        if (c0 + u >= nch) break;  // uniform
        const float Mn = fmaxf(M, mc[u]);
        const float keep = M == -INFINITY ? 0.f : __expf(M - Mn);
        const float w = mc[u] == -INFINITY ? 0.f : __expf(mc[u] - Mn);
        Ls = Ls * keep + w * lc[u];
        acc = acc * keep + w * oc[u];
        M = Mn;
      }
    }
    a.o[bh * D + d] = r16(acc / Ls);
  }
  __syncthreads();  // every thread has read the partials
  uint32_t* pw = reinterpret_cast<uint32_t*>(a.partial + bh * a.max_chunks * kStride);
  for (uint32_t i = threadIdx.x; i < nch * kStride; i += W * 64u) st_agent_u32(pw + i, 0u);
}

// ---------------------------------------------------------------- prefill
// Causal (or full) attention of Lq queries, the last Lq positions of an
// L-token paged sequence: one lane group per (query, head), keys in order,
// online softmax in fp32, sm_scale applied in fp32.
template <int D>
__global__ __launch_bounds__(256) void gen_prefill_kernel(PrefillArgs a) {
  constexpr uint32_t N = D / 8, QPB = 256u / N;
  const uint32_t l = threadIdx.x % N;
  const uint32_t qi = blockIdx.x * QPB + threadIdx.x / N;
  const uint32_t h = blockIdx.y;
  const uint32_t hkv = h / (a.Hq / a.H);
  const uint32_t S = a.g.kv / (a.H * D);  // tokens per page
  const uint32_t off = a.L - a.Lq;
  const bool live = qi < a.Lq;
  const uint32_t qpos = off + (live ? qi : a.Lq - 1u);
  const uint32_t kend = a.causal ? qpos + 1u : a.L;
  // keys the block walks: up to its last query's
  uint32_t qlast = blockIdx.x * QPB + QPB - 1u;
  if (qlast >= a.Lq) qlast = a.Lq - 1u;
  const uint32_t block_kend = a.causal ? off + qlast + 1u : a.L;
  const H8 q = live ? ld16(a.q + ((size_t)qi * a.Hq + h) * D + l * kVec) : H8{};
  float m = -INFINITY, lsum = 0.f, o[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) o[j] = 0.f;
  for (uint32_t k = 0; k < block_kend; ++k) {
    const uint32_t phys = (uint32_t)a.kv_indices[k / S];
    const H8 kk = ld16(a.kv + elem_off(a.g, phys, 0, hkv, k % S) + l * kVec);
    const H8 vv = ld16(a.kv + elem_off(a.g, phys, 1, hkv, k % S) + l * kVec);
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kVec; ++j) acc = acc + (float)q.v[j] * (float)kk.v[j];
    const float x = grp_sum<N>(acc) * a.sm_scale;
    if (k < kend) {
      const float mn = fmaxf(m, x);
      const float c = m == -INFINITY ? 0.f : __expf(m - mn);
      const float p = __expf(x - mn);
      lsum = lsum * c + p;
#pragma unroll
      for (int j = 0; j < kVec; ++j) o[j] = o[j] * c + p * (float)vv.v[j];
      m = mn;
    }
  }
  if (live) {
    H8 out;
#pragma unroll
    for (int j = 0; j < kVec; ++j) out.v[j] = r16(o[j] / lsum);
    st16(a.o + ((size_t)qi * a.Hq + h) * D + l * kVec, out);
  }
}

}  // namespace

// ---------------------------------------------------------------- launchers
// head_dim dispatch (64, 128, 256), as the reference's SWITCH_HEAD_DIM
#define AOAKV_GEN_D(D_, ...)      \
  switch (D_) {                   \
    case 64: {                    \
      constexpr int D = 64;       \
      __VA_ARGS__;                \
      break;                      \
    }                             \
    case 128: {                   \
      constexpr int D = 128;      \
      __VA_ARGS__;                \
      break;                      \
    }                             \
    case 256: {                   \
      constexpr int D = 256;      \
      __VA_ARGS__;                \
      break;                      \
    }                             \
    default:                      \
      return hipErrorInvalidValue; \
  }

hipError_t launch_gen_append_prefill(const AppendPrefillArgs& a, uint32_t D_, hipStream_t s) {
  const uint32_t L = (a.num_pages - 1u) * a.S + a.last_page_len;
  AppendPrefillArgs b = a;
  b.first_page = (L - a.N) / a.S;
  AOAKV_GEN_D(D_, {
    const uint32_t hpb = 256u / (D / 8);
    dim3 grid(a.num_pages - b.first_page, (a.H + hpb - 1) / hpb);
    hipLaunchKernelGGL(gen_append_prefill_kernel<D>, grid, dim3(256), 0, s, b);
  })
  return hipGetLastError();
}

hipError_t launch_gen_append_decode(const AppendDecodeArgs& a, uint32_t batch, uint32_t D_,
                                    hipStream_t s) {
  AOAKV_GEN_D(D_, {
    const uint32_t hpb = 256u / (D / 8);
    const uint32_t kv_blocks = (a.H + hpb - 1) / hpb;
    if (a.rope) {
      const uint32_t q_blocks = (a.Hq + hpb - 1) / hpb;
      hipLaunchKernelGGL((gen_append_decode_kernel<D, true>), dim3(batch, kv_blocks + q_blocks),
                         dim3(256), 0, s, a);
    } else {
      hipLaunchKernelGGL((gen_append_decode_kernel<D, false>), dim3(batch, kv_blocks), dim3(256),
                         0, s, a);
    }
  })
  return hipGetLastError();
}

hipError_t launch_gen_rope(const RopeArgs& a, uint32_t D_, hipStream_t s) {
  if (a.N == 0u) return hipSuccess;
  AOAKV_GEN_D(D_, hipLaunchKernelGGL(gen_rope_kernel<D>, dim3(a.N), dim3(256), 0, s, a))
  return hipGetLastError();
}

hipError_t launch_gen_estimate(const EstimateArgs& a, uint32_t batch, uint32_t max_pages,
                               uint32_t D_, hipStream_t s) {
  const dim3 grid((max_pages + kGenPagesPerBlock - 1) / kGenPagesPerBlock, a.Hkv, batch);
  const uint32_t group = a.Hq / a.Hkv;
  AOAKV_GEN_D(D_, {
    switch (group) {
      case 1: hipLaunchKernelGGL((gen_estimate_kernel<D, 1>), grid, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((gen_estimate_kernel<D, 2>), grid, dim3(256), 0, s, a); break;
      case 4: hipLaunchKernelGGL((gen_estimate_kernel<D, 4>), grid, dim3(256), 0, s, a); break;
      case 8: hipLaunchKernelGGL((gen_estimate_kernel<D, 8>), grid, dim3(256), 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
  })
  return hipGetLastError();
}

hipError_t launch_gen_decode(const DecodeArgs& a, uint32_t batch, uint32_t D_, hipStream_t s) {
  // 8 waves (a page each) while the grid fits the GPU's 256 CUs once over
  // (32k context, budget 2048: head dim 256 19.9 -> 15.2 us, page size 32
  // 18.4 -> 14.4); with more workgroups, 4 waves, of which more fit per CU
  // (page size 8, 1,024 workgroups: 15.5 us with 4 waves, 30.9 with 8).
  // Without GQA the K/V loads stream (non-temporal): over 32 rotated layers
  // head dim 64 23.1 -> 22.2 us per layer (scores + decode), 256 34.4 ->
  // 32.5, page size 8 41.4 -> 39.1, page size 32 27.9 -> 27.0, with the
  // scoring's metadata streamed too
  const bool wide = (size_t)a.max_chunks * a.Hq * batch <= 256u;
  const bool stream = a.Hq == a.Hkv;
  const dim3 grid(a.max_chunks, a.Hq, batch);
  AOAKV_GEN_D(D_, {
    if (wide && stream)
      hipLaunchKernelGGL((gen_decode_kernel<D, 8, true>), grid, dim3(512), 0, s, a);
    else if (wide)
      hipLaunchKernelGGL((gen_decode_kernel<D, 8, false>), grid, dim3(512), 0, s, a);
    else if (stream)
      hipLaunchKernelGGL((gen_decode_kernel<D, 4, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((gen_decode_kernel<D, 4, false>), grid, dim3(256), 0, s, a);
  })
  return hipGetLastError();
}

hipError_t launch_gen_prefill(const PrefillArgs& a, uint32_t D_, hipStream_t s) {
  AOAKV_GEN_D(D_, {
    const uint32_t qpb = 256u / (D / 8);
    hipLaunchKernelGGL(gen_prefill_kernel<D>, dim3((a.Lq + qpb - 1) / qpb, a.Hq), dim3(256), 0,
                       s, a);
  })
  return hipGetLastError();
}

#undef AOAKV_GEN_D

}  // namespace aoakv
