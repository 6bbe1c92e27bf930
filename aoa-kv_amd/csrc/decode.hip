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
// workgroup to arrive at a per-head counter, which it resets to zero.
#include "kernels.hpp"

namespace aoakv {

constexpr int kThreads = 256;
constexpr int kEstPagesPerWave = 32;                     // 8 steps x 4 rows
constexpr int kEstPagesPerBlock = kEstPagesPerWave * 4;  // 128
constexpr int kTopkMaxLds = 4096;                        // keys staged in LDS
constexpr int kDecPagesPerWave = 2;
constexpr int kDecPagesPerBlock = kDecPagesPerWave * 4;  // 8
constexpr int kPartialStride = kHeadDim + 4;             // o[128], m, l, pad

// ======================================================================
// top-k selection for one (sequence, kv head), one 256-thread block
// ======================================================================

struct TopkShared {
  uint32_t keys[kTopkMaxLds];
  uint32_t hist[256];
  uint32_t red[8];
  uint32_t bin, above;
  uint32_t wsum[4][2];
};

__device__ inline uint32_t wave_excl_count(bool flag, uint64_t& mask) {
  mask = __ballot(flag);
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Selects k of P pages from fp32 `scores` (filter_util.py:373-380): with
// `fixed`, pages 0 and P-1 always; the rest by descending score, ties to the
// lower page index.  Writes kv_ids[page] of the selected pages to out[] in
// ascending page order.  Key order = float order (order_key).
__device__ void topk_block(const float* __restrict__ scores, uint32_t P, uint32_t k, bool fixed,
                           const int32_t* __restrict__ kv_ids, int32_t* __restrict__ out,
                           TopkShared& sh) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = __lane_id();
  const uint32_t wave = tid / kWave;
  const bool in_lds = P <= (uint32_t)kTopkMaxLds;

  if (k >= P) {  // everything selected
    for (uint32_t i = tid; i < P; i += kThreads) out[i] = kv_ids[i];
    return;
  }
  auto forced = [&](uint32_t i) { return fixed && (i == 0u || i == P - 1u); };
  auto key_at = [&](uint32_t i) -> uint32_t {
    return in_lds ? sh.keys[i] : order_key(__builtin_nontemporal_load(scores + i));
  };

  // stage keys, min / max over the free (non-forced) pages
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
  for (uint32_t i = tid; i < P; i += kThreads) {
    uint32_t key = order_key(scores[i]);
    if (in_lds) sh.keys[i] = key;
    if (!forced(i)) {
      kmin = key < kmin ? key : kmin;
      kmax = key > kmax ? key : kmax;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t a = __shfl_xor(kmin, off);
    uint32_t b = __shfl_xor(kmax, off);
    kmin = a < kmin ? a : kmin;
    kmax = b > kmax ? b : kmax;
  }
  if (lane == 0) {
    sh.red[wave] = kmin;
    sh.red[4 + wave] = kmax;
  }
  __syncthreads();
  kmin = sh.red[0];
  kmax = sh.red[4];
  for (int w = 1; w < 4; ++w) {
    kmin = sh.red[w] < kmin ? sh.red[w] : kmin;
    kmax = sh.red[4 + w] > kmax ? sh.red[4 + w] : kmax;
  }
  const uint32_t nforced = fixed ? (P == 1u ? 1u : 2u) : 0u;
  uint32_t kr = k - nforced;  // >= 1 because k >= 3 whenever k < P

  // radix select of the kr-th largest free key, digits of the key offset
  // (key - kmin) from its top set bit down (the offsets of one head's scores
  // span a narrow range, so the first digit already spreads the histogram)
  const uint32_t range = kmax - kmin;
  uint64_t prefix = 0;
  int hi = range == 0u ? 0 : 32 - __builtin_clz(range);
  while (hi > 0) {
    const int w = hi < 8 ? hi : 8;
    const int sh_ = hi - w;
    for (uint32_t i = tid; i < 256u; i += kThreads) sh.hist[i] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < P; i += kThreads) {
      if (forced(i)) continue;
      uint64_t rel = (uint64_t)(key_at(i) - kmin);
      if ((rel >> hi) == (prefix >> hi)) atomicAdd(&sh.hist[(uint32_t)(rel >> sh_) & ((1u << w) - 1u)], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      // lane L holds bins 255-4L .. 252-4L (descending)
      uint32_t c[4], s4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = sh.hist[255u - 4u * lane - j];
        s4 += c[j];
      }
      uint32_t incl = s4;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        uint32_t t = __shfl_up(incl, off);
        if ((int)lane >= off) incl += t;
      }
      uint32_t excl = incl - s4;
      if (excl < kr && kr <= incl) {
        uint32_t cc = excl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (cc + c[j] >= kr) {
            sh.bin = 255u - 4u * lane - j;
            sh.above = cc;
            break;
          }
          cc += c[j];
        }
      }
    }
    __syncthreads();
    prefix |= (uint64_t)sh.bin << sh_;
    kr -= sh.above;
    hi = sh_;
    __syncthreads();
  }
  const uint32_t T = kmin + (uint32_t)prefix;  // key of the k-th free page
  const uint32_t take_eq = kr;                 // pages with key == T to take

  // compaction in ascending page order, 256 pages per round
  uint32_t base_sel = 0, base_eq = 0;
  for (uint32_t r0 = 0; r0 < P; r0 += kThreads) {
    const uint32_t i = r0 + tid;
    bool valid = i < P;
    uint32_t key = valid ? key_at(i) : 0u;
    bool f = valid && forced(i);
    bool eq = valid && !f && key == T;
    bool gt = valid && !f && key > T;
    uint64_t m_eq, m_sel;
    uint32_t eq_rank = wave_excl_count(eq, m_eq);
    if (lane == 0) sh.wsum[wave][0] = (uint32_t)__popcll(m_eq);
    __syncthreads();
    uint32_t eq_before = base_eq;
    for (uint32_t w = 0; w < wave; ++w) eq_before += sh.wsum[w][0];
    bool take = f || gt || (eq && eq_before + eq_rank < take_eq);
    uint32_t sel_rank = wave_excl_count(take, m_sel);
    if (lane == 0) sh.wsum[wave][1] = (uint32_t)__popcll(m_sel);
    __syncthreads();
    uint32_t sel_before = base_sel;
    for (uint32_t w = 0; w < wave; ++w) sel_before += sh.wsum[w][1];
    if (take) out[sel_before + sel_rank] = kv_ids[i];
    for (uint32_t w = 0; w < 4; ++w) {
      base_eq += sh.wsum[w][0];
      base_sel += sh.wsum[w][1];
    }
    __syncthreads();
  }
}

// ======================================================================
// page scores (+ optional fused top-k)
// ======================================================================


template <int GROUP>
__global__ __launch_bounds__(kThreads) void estimate_kernel(EstimateArgs a) {
  __shared__ TopkShared sh;
  __shared__ uint32_t s_last;
  const uint32_t lane = __lane_id();
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t row = lane / kLanesPerRow;
  const uint32_t l16 = lane % kLanesPerRow;
  const uint32_t b = blockIdx.z, h = blockIdx.y, chunk = blockIdx.x;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  uint32_t P = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  if (P > a.score_stride) P = a.score_stride;  // never write past a score row
  if (chunk * kEstPagesPerBlock >= P) return;  // uniform per block
  const uint32_t S = a.S;
  const uint32_t mbeg = (uint32_t)a.meta_indptr[b];
  const uint32_t d0 = l16 * kVec;
  const bool value_aware = (a.flags & 1u) != 0u;

  float qf[GROUP][kVec];
#pragma unroll
  for (int g = 0; g < GROUP; ++g) {
    H8 qq = ld16(a.q + ((size_t)b * a.Hq + h * GROUP + g) * kHeadDim + d0);
#pragma unroll
    for (int j = 0; j < kVec; ++j) qf[g][j] = (float)qq.v[j];
  }

  const uint32_t page0 = chunk * kEstPagesPerBlock + wave * kEstPagesPerWave;
  constexpr int kSteps = kEstPagesPerWave / 4;
  H8 kmx[kSteps], kmn[kSteps];
  f16 lvn[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const uint32_t p = page0 + s * 4 + row;
    if (p < P) {
      const uint32_t mp = (uint32_t)a.meta_indices[mbeg + p / S];
      const size_t off = elem_off(a.g, mp, 0, h, p % S) + d0;
      kmx[s] = ld16(a.meta + off);
      kmn[s] = ld16(a.meta + off + a.g.kv);
      if (value_aware)
        lvn[s] = a.v_log_norm[(size_t)(uint32_t)a.kv_indices[pbeg + p] * a.Hkv + h];
    }
  }
  float* out = a.scores + ((size_t)b * a.Hkv + h) * a.score_stride;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const uint32_t p = page0 + s * 4 + row;
    float x[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        float u = qf[g][j] * (float)kmx[s].v[j];
        float w = qf[g][j] * (float)kmn[s].v[j];
        acc = acc + fmaxf(u, w);
      }
      x[g] = row_sum16(acc);
    }
    float score;
    if (value_aware) {
      // 2 * (bound / sqrt(d)), logsumexp over the group, + 2 * log-norm
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
      score = lse + 2.0f * (float)lvn[s];
    } else {
      score = x[0];
#pragma unroll
      for (int g = 1; g < GROUP; ++g) score = score + x[g];
    }
    if (p < P && l16 == 0u) out[p] = score;
  }

  if (a.sel == nullptr) return;
  // ---- fused top-k: the last block of this (sequence, head) selects
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t nch = (P + kEstPagesPerBlock - 1) / kEstPagesPerBlock;
    const uint32_t prev = atomicAdd(&a.counters[b * a.Hkv + h], 1u);
    s_last = prev == nch - 1u ? 1u : 0u;
  }
  __syncthreads();
  if (s_last == 0u) return;
  __threadfence();
  const uint32_t L = (P - 1u) * S + (uint32_t)a.kv_last_page_len[b];
  const uint32_t budget = a.token_budgets ? (uint32_t)a.token_budgets[b] : a.token_budget;
  uint32_t k = num_selected_pages(L, budget, S, P);
  if (k > a.sel_stride) k = a.sel_stride;  // never write past a selection row
  topk_block(out, P, k, (a.flags & 2u) != 0u, a.kv_indices + pbeg,
             a.sel + ((size_t)b * a.Hkv + h) * a.sel_stride, sh);
  if (threadIdx.x == 0) a.counters[b * a.Hkv + h] = 0u;
}


__global__ __launch_bounds__(kThreads) void topk_kernel(TopkArgs a) {
  __shared__ TopkShared sh;
  const uint32_t h = blockIdx.x, b = blockIdx.y;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  uint32_t P = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  if (P == 0u) return;
  if (P > a.score_stride) P = a.score_stride;
  const uint32_t L = (P - 1u) * a.S + (uint32_t)a.kv_last_page_len[b];
  const uint32_t budget = a.token_budgets ? (uint32_t)a.token_budgets[b] : a.token_budget;
  uint32_t k = num_selected_pages(L, budget, a.S, P);
  if (k > a.sel_stride) k = a.sel_stride;
  topk_block(a.scores + ((size_t)b * a.Hkv + h) * a.score_stride, P, k, (a.flags & 2u) != 0u,
             a.kv_indices + pbeg, a.sel + ((size_t)b * a.Hkv + h) * a.sel_stride, sh);
}

// ======================================================================
// sparse decode attention, split-K over pages with a fused merge
// ======================================================================


__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeArgs a) {
  __shared__ float s_o[4][kHeadDim];
  __shared__ float s_ml[4][2];
  __shared__ uint32_t s_last;
  const uint32_t lane = __lane_id();
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t row = lane / kLanesPerRow;
  const uint32_t l16 = lane % kLanesPerRow;
  const uint32_t b = blockIdx.z, hq = blockIdx.y, chunk = blockIdx.x;
  const uint32_t hkv = hq / (a.Hq / a.Hkv);
  const uint32_t S = a.S;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  const uint32_t lpl = (uint32_t)a.kv_last_page_len[b];
  if (P == 0u || lpl == 0u || lpl > S) return;  // malformed page table
  uint32_t npages = P;
  if (a.sel != nullptr) {
    const uint32_t budget = a.token_budgets ? (uint32_t)a.token_budgets[b] : a.token_budget;
    npages = num_selected_pages((P - 1u) * S + lpl, budget, S, P);
    if (npages > a.sel_stride) npages = a.sel_stride;
  }
  // the grid holds max_chunks blocks per head; never index partials past it
  if (npages > a.max_chunks * kDecPagesPerBlock) npages = a.max_chunks * kDecPagesPerBlock;
  const uint32_t nch = (npages + kDecPagesPerBlock - 1) / kDecPagesPerBlock;
  if (chunk >= nch) return;  // uniform per block
  const uint32_t last_phys = (uint32_t)a.kv_indices[pbeg + P - 1u];
  const uint32_t d0 = l16 * kVec;
  const size_t bh = (size_t)b * a.Hq + hq;

  float qf[kVec];
  {
    H8 qq = ld16(a.q + bh * kHeadDim + d0);
#pragma unroll
    for (int j = 0; j < kVec; ++j) qf[j] = (float)qq.v[j];
  }

  // ---- issue all loads of this wave's pages
  H8 kk[kDecPagesPerWave][4], vv[kDecPagesPerWave][4];
  uint32_t ntok[kDecPagesPerWave];
#pragma unroll
  for (int s = 0; s < kDecPagesPerWave; ++s) {
    const uint32_t idx = chunk * kDecPagesPerBlock + wave * kDecPagesPerWave + s;
    ntok[s] = 0u;
    if (idx < npages) {
      const uint32_t phys = a.sel ? (uint32_t)a.sel[((size_t)b * a.Hkv + hkv) * a.sel_stride + idx]
                                  : (uint32_t)a.kv_indices[pbeg + idx];
      ntok[s] = phys == last_phys ? lpl : S;
      const size_t kbase = elem_off(a.g, phys, 0, hkv, 0) + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t t = i * 4 + row;
        kk[s][i] = ld16(a.kv + kbase + (size_t)t * a.g.tok);
        vv[s][i] = ld16(a.kv + kbase + a.g.kv + (size_t)t * a.g.tok);
      }
    }
  }

  // ---- logits: fp16(q.k), then fp16(. / sqrt(d))  (quest_attention.py:265-268)
  float x[kDecPagesPerWave][4];
  float mloc = -INFINITY;
#pragma unroll
  for (int s = 0; s < kDecPagesPerWave; ++s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kVec; ++j) acc = acc + qf[j] * (float)kk[s][i].v[j];
      acc = row_sum16(acc);
      const float lg = (float)r16((float)r16(acc) / kSqrtHeadDim);
      const uint32_t t = i * 4 + row;
      x[s][i] = t < ntok[s] ? lg : -INFINITY;
      mloc = fmaxf(mloc, x[s][i]);
    }
  }
  const float m = cross_row_max(mloc);
  float lsum = 0.f;
  float o[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) o[j] = 0.f;
  if (m != -INFINITY) {
#pragma unroll
    for (int s = 0; s < kDecPagesPerWave; ++s) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __expf(x[s][i] - m);
        lsum = lsum + p;
#pragma unroll
        for (int j = 0; j < kVec; ++j) o[j] = o[j] + p * (float)vv[s][i].v[j];
      }
    }
  }
  lsum = cross_row_sum(lsum);
#pragma unroll
  for (int j = 0; j < kVec; ++j) o[j] = cross_row_sum(o[j]);

  // ---- combine the 4 waves of the block in LDS
  if (row == 0u) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) s_o[wave][d0 + j] = o[j];
    if (l16 == 0u) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = lsum;
    }
  }
  __syncthreads();
  float* part = a.partial + (bh * a.max_chunks + chunk) * kPartialStride;
  if (threadIdx.x < (uint32_t)kHeadDim) {
    const uint32_t d = threadIdx.x;
    float M = fmaxf(fmaxf(s_ml[0][0], s_ml[1][0]), fmaxf(s_ml[2][0], s_ml[3][0]));
    float acc = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = s_ml[w][0] == -INFINITY ? 0.f : __expf(s_ml[w][0] - M);
      acc = acc + sc * s_o[w][d];
      l = l + sc * s_ml[w][1];
    }
    part[d] = acc;
    if (d == 0u) {
      part[kHeadDim] = M;
      part[kHeadDim + 1] = l;
    }
  }

  // ---- the last block of this (sequence, head) merges the chunks
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(&a.counters[bh], 1u);
    s_last = prev == nch - 1u ? 1u : 0u;
  }
  __syncthreads();
  if (s_last == 0u) return;
  __threadfence();
  if (threadIdx.x < (uint32_t)kHeadDim) {
    const uint32_t d = threadIdx.x;
    const float* base = a.partial + bh * a.max_chunks * kPartialStride;
    float M = -INFINITY;
    for (uint32_t c = 0; c < nch; ++c) M = fmaxf(M, base[c * kPartialStride + kHeadDim]);
    float acc = 0.f, l = 0.f;
    for (uint32_t c = 0; c < nch; ++c) {
      const float* pc = base + c * kPartialStride;
      const float sc = __expf(pc[kHeadDim] - M);
      acc = acc + sc * pc[d];
      l = l + sc * pc[kHeadDim + 1];
    }
    a.o[bh * kHeadDim + d] = r16(acc / l);
  }
  if (threadIdx.x == 0) a.counters[bh] = 0u;
}

__global__ void fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------- launchers

hipError_t launch_estimate(const EstimateArgs& a, uint32_t batch, uint32_t max_pages,
                           hipStream_t s) {
  dim3 grid((max_pages + kEstPagesPerBlock - 1) / kEstPagesPerBlock, a.Hkv, batch);
  switch (a.Hq / a.Hkv) {
    case 1: hipLaunchKernelGGL(estimate_kernel<1>, grid, dim3(kThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL(estimate_kernel<2>, grid, dim3(kThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL(estimate_kernel<4>, grid, dim3(kThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL(estimate_kernel<8>, grid, dim3(kThreads), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_topk(const TopkArgs& a, uint32_t batch, hipStream_t s) {
  hipLaunchKernelGGL(topk_kernel, dim3(a.Hkv, batch), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, uint32_t batch, hipStream_t s) {
  dim3 grid(a.max_chunks, a.Hq, batch);
  hipLaunchKernelGGL(decode_kernel, grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

uint32_t decode_chunks(uint32_t max_sel_pages) {
  return (max_sel_pages + kDecPagesPerBlock - 1) / kDecPagesPerBlock;
}
uint32_t partial_stride() { return kPartialStride; }

}  // namespace aoakv
