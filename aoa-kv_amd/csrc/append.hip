// Paged KV append with AOA-KV metadata maintenance (gfx950).
//
// Replaces the reference's AppendPagedKVCachePrefillKernel and
// AppendPagedKVCacheDecodeKernel (kernels/aoa_kv/kernels/include/decode/
// decode_page.cuh:398-692) with the simulation's semantics
// (filtering/filter_util.py:555-638, 669-716, 758-834):
//   * per page and head: Kmax / Kmin (exact fp16 min/max),
//   * V̄ = page mean of V (fp32 sum in token order, one rounding) for a page
//     filled from empty, the fp16 running mean for tokens added to a page
//     that already holds tokens,
//   * log-norm of V̄ for EVERY page, the partial last page included (the
//     reference kernel only writes full pages and reads them at the wrong
//     index, decode_attn.cuh:185-190).
//
// Work mapping: a workgroup of 4 waves covers one page x 16 heads; each
// wave covers 4 heads, one 16-lane DPP row per head, 8 dims per lane.  A
// wave's 16-byte loads of one token read 4 consecutive heads = 1 KB
// contiguous from the NHD input.
#include "kernels.hpp"

namespace aoakv {

constexpr int kHeadsPerWave = 4;
constexpr int kHeadsPerBlock = 16;


__global__ __launch_bounds__(256) void append_prefill_kernel(AppendPrefillArgs a) {
  const uint32_t lane = __lane_id();
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t row = lane / kLanesPerRow;
  const uint32_t l16 = lane % kLanesPerRow;
  const uint32_t h = blockIdx.y * kHeadsPerBlock + wave * kHeadsPerWave + row;
  const uint32_t p = a.first_page + blockIdx.x;
  if (h >= a.H || p >= a.num_pages) return;  // whole rows exit together

  const uint32_t S = a.S;
  const uint32_t L = (a.num_pages - 1u) * S + a.last_page_len;
  const uint32_t start = L - a.N;  // first appended position
  const uint32_t e0 = start > p * S ? start - p * S : 0u;
  const uint32_t e1 = (L - p * S) < S ? (L - p * S) : S;
  const uint32_t phys = (uint32_t)a.kv_indices[p];
  const uint32_t mpage = (uint32_t)a.meta_indices[p / S];
  const uint32_t ment = p % S;
  const uint32_t d0 = l16 * kVec;

  f16* kmax_p = a.meta + elem_off(a.g, mpage, 0, h, ment) + d0;
  f16* kmin_p = a.meta + elem_off(a.g, mpage, 1, h, ment) + d0;
  f16* vbar_p = a.v_mean + ((size_t)phys * a.H + h) * kHeadDim + d0;

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

  const size_t in_row = (size_t)a.H * kHeadDim;
  const f16* kin = a.k + (size_t)(p * S + e0 - start) * in_row + (size_t)h * kHeadDim + d0;
  const f16* vin = a.v + (size_t)(p * S + e0 - start) * in_row + (size_t)h * kHeadDim + d0;
  f16* kout = a.kv + elem_off(a.g, phys, 0, h, e0) + d0;
  f16* vout = a.kv + elem_off(a.g, phys, 1, h, e0) + d0;

  const uint32_t n = e1 - e0;
  if (e0 == 0u) {
    // page filled from empty: V̄ = mean over its tokens (compute_page_v_mean)
#pragma unroll 4
    for (uint32_t i = 0; i < n; ++i) {
      H8 kk = ld16(kin + i * in_row);
      H8 vv = ld16(vin + i * in_row);
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        kmax.v[j] = kk.v[j] > kmax.v[j] ? kk.v[j] : kmax.v[j];
        kmin.v[j] = kk.v[j] < kmin.v[j] ? kk.v[j] : kmin.v[j];
        vsum[j] = vsum[j] + (float)vv.v[j];
      }
      st16(kout + (size_t)i * a.g.tok, kk);
      st16(vout + (size_t)i * a.g.tok, vv);
    }
#pragma unroll
    for (int j = 0; j < kVec; ++j) vbar.v[j] = r16(vsum[j] / (float)n);
  } else {
    // tokens added to a page that already holds e0 tokens: running mean
    for (uint32_t i = 0; i < n; ++i) {
      H8 kk = ld16(kin + i * in_row);
      H8 vv = ld16(vin + i * in_row);
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        kmax.v[j] = kk.v[j] > kmax.v[j] ? kk.v[j] : kmax.v[j];
        kmin.v[j] = kk.v[j] < kmin.v[j] ? kk.v[j] : kmin.v[j];
        vbar.v[j] = running_mean(vbar.v[j], vv.v[j], e0 + i);
      }
      st16(kout + (size_t)i * a.g.tok, kk);
      st16(vout + (size_t)i * a.g.tok, vv);
    }
  }
  st16(kmax_p, kmax);
  st16(kmin_p, kmin);
  st16(vbar_p, vbar);
  f16 lvn = log_norm_row(vbar, l16);
  if (l16 == 0u) a.v_log_norm[(size_t)phys * a.H + h] = lvn;
}


// One new token per sequence (update_page_filters / update_mean_page_filters,
// filter_util.py:681-716, 758-795).  With ROPE the block rows of grid.y past
// the kv heads' rotate q in place, and k is rotated (in place, and as stored)
// before the append: RoPE + append + metadata in one launch, the reference's
// apply_rope_in_place then append_kv_cache_decode (QuestAttention.py:98-111).
// The new token sits at position L - 1 of its sequence (L counts it).
template <bool ROPE>
__global__ __launch_bounds__(256) void append_decode_kernel(AppendDecodeArgs a) {
  const uint32_t lane = __lane_id();
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t row = lane / kLanesPerRow;
  const uint32_t l16 = lane % kLanesPerRow;
  const uint32_t b = blockIdx.x;
  const uint32_t kv_blocks = (a.H + kHeadsPerBlock - 1) / kHeadsPerBlock;
  const bool q_block = ROPE && blockIdx.y >= kv_blocks;  // uniform per block
  const uint32_t h = (q_block ? blockIdx.y - kv_blocks : blockIdx.y) * kHeadsPerBlock +
                     wave * kHeadsPerWave + row;
  if (h >= (q_block ? a.Hq : a.H)) return;

  const uint32_t S = a.S;
  const uint32_t pbeg = (uint32_t)a.kv_indptr[b];
  const uint32_t P = (uint32_t)a.kv_indptr[b + 1] - pbeg;
  const uint32_t lpl = (uint32_t)a.kv_last_page_len[b];
  if (P == 0u || lpl == 0u || lpl > S) return;  // malformed page table: nothing to do
  RopeTable rt;
  if constexpr (ROPE) {
    rt = rope_table((P - 1u) * S + lpl - 1u, l16, a.rope_f.f);
    if (q_block) {
      f16* qp = a.q + ((size_t)b * a.Hq + h) * kHeadDim + l16 * kVec;
      st16(qp, rope_row(ld16(qp), rt, l16));
      return;
    }
  }
  const uint32_t e = lpl - 1u;  // entry of the new token
  const uint32_t p = P - 1u;
  const uint32_t phys = (uint32_t)a.kv_indices[pbeg + p];
  const uint32_t mpage = (uint32_t)a.meta_indices[(uint32_t)a.meta_indptr[b] + p / S];
  const uint32_t ment = p % S;
  const uint32_t d0 = l16 * kVec;

  f16* kmax_p = a.meta + elem_off(a.g, mpage, 0, h, ment) + d0;
  f16* kmin_p = a.meta + elem_off(a.g, mpage, 1, h, ment) + d0;
  f16* vbar_p = a.v_mean + ((size_t)phys * a.H + h) * kHeadDim + d0;

  const size_t in_off = ((size_t)b * a.H + h) * kHeadDim + d0;
  H8 kk = ld16(a.k + in_off);
  H8 vv = ld16(a.v + in_off);
  if constexpr (ROPE) {
    kk = rope_row(kk, rt, l16);
    st16(a.k + in_off, kk);
  }
  H8 kmax, kmin, vbar;
  if (e == 0u) {  // new page: max = min = k, V̄ = v
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
  f16 lvn = log_norm_row(vbar, l16);
  if (l16 == 0u) a.v_log_norm[(size_t)phys * a.H + h] = lvn;
}

hipError_t launch_append_prefill(const AppendPrefillArgs& a, hipStream_t s) {
  const uint32_t L = (a.num_pages - 1u) * a.S + a.last_page_len;
  const uint32_t first_page = (L - a.N) / a.S;
  AppendPrefillArgs b = a;
  b.first_page = first_page;
  dim3 grid(a.num_pages - first_page, (a.H + kHeadsPerBlock - 1) / kHeadsPerBlock);
  hipLaunchKernelGGL(append_prefill_kernel, grid, dim3(256), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_append_decode(const AppendDecodeArgs& a, uint32_t batch, hipStream_t s) {
  const uint32_t kv_blocks = (a.H + kHeadsPerBlock - 1) / kHeadsPerBlock;
  if (a.rope) {
    const uint32_t q_blocks = (a.Hq + kHeadsPerBlock - 1) / kHeadsPerBlock;
    hipLaunchKernelGGL(append_decode_kernel<true>, dim3(batch, kv_blocks + q_blocks), dim3(256),
                       0, s, a);
  } else {
    hipLaunchKernelGGL(append_decode_kernel<false>, dim3(batch, kv_blocks), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

// In-place RoPE of q [N, Hq, D] and k [N, Hkv, D], token n at position
// past + n (apply_rope_in_place, page.cu:224-265).  A block takes one token:
// each lane computes the cos / sin of its 8 dims once and its row rotates
// heads row, row + 16, ... of q then k.
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const uint32_t lane = __lane_id();
  const uint32_t l16 = lane % kLanesPerRow;
  const uint32_t r = threadIdx.x / kLanesPerRow;  // 16 rows per block
  const uint32_t n = blockIdx.x;
  const RopeTable rt = rope_table(a.past + n, l16, a.rope_f.f);
  for (uint32_t h = r; h < a.Hq + a.Hkv; h += 16u) {
    f16* p = h < a.Hq ? a.q + ((size_t)n * a.Hq + h) * kHeadDim
                      : a.k + ((size_t)n * a.Hkv + (h - a.Hq)) * kHeadDim;
    p += l16 * kVec;
    st16(p, rope_row(ld16(p), rt, l16));
  }
}

hipError_t launch_rope(const RopeArgs& a, hipStream_t s) {
  if (a.N == 0u) return hipSuccess;
  hipLaunchKernelGGL(rope_kernel, dim3(a.N), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace aoakv
