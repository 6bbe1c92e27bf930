// Dense causal prefill over the paged cache, gfx950 MFMA (fp16 in, fp32 acc).
//
// Replaces BatchPrefillWithPagedKVCacheKernel (kernels/aoa_kv/kernels/include/
// prefill/prefill.cuh:688-870) for one sequence: o = softmax(q k^T / sqrt(d)) v
// with query i (position L - qo_len + i) attending keys 0 .. L - qo_len + i.
//
// Formulation: each wave owns 32 queries and computes the transposed scores
// S^T = K Q^T with v_mfma_f32_32x32x16_f16 (keys on the MFMA rows, queries on
// the columns).  In the 32x32 accumulator lane l holds column l%32, so every
// lane holds the scores of ONE query -- its own -- for 16 of the tile's 32
// keys (the other 16 sit in lane l^32).  The softmax row statistics are
// therefore per lane (plus one exchange with lane l^32), and the fp16
// probabilities already sit in the B-operand layout of O^T += V^T P^T, so P
// never goes through LDS.  Lane layouts (checked on the hardware):
//   A: lane l -> row l%32, 8 k-values;  B: lane l -> column l%32, 8 k-values,
//   A and B elements with the same (l/32, j) share a k;
//   C: register i of lane l -> row 8*(i/4) + 4*(l/32) + i%4, column l%32.
//
// Block = 4 waves = 128 queries of one head; K/V tiles of 64 keys (4 pages)
// are gathered from the page table into LDS (K row-major, V transposed) with
// the next tile's loads in flight during the current tile's MFMAs.
#include "kernels.hpp"

namespace aoakv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kPfThreads = 256;
constexpr int kPfQueriesPerWave = 32;
constexpr int kPfQueriesPerBlock = 128;
constexpr int kPfTileKeys = 64;
constexpr int kKRow = kHeadDim + 8;    // LDS row of K (halfs), padded against bank conflicts
constexpr int kVRow = kPfTileKeys + 8; // LDS row of V^T (halfs)
constexpr float kLog2e = 1.4426950408889634f;

__device__ inline floatx16 mfma32(const half8& a, const half8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// row of accumulator register i for lane group g
__device__ inline int crow(int i, int g) { return 8 * (i / 4) + 4 * g + (i % 4); }

__global__ __launch_bounds__(kPfThreads) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) f16 sK[kPfTileKeys * kKRow];
  __shared__ __attribute__((aligned(16))) f16 sVt[kHeadDim * kVRow];
  const int tid = threadIdx.x;
  const int lane = (int)__lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane / 32;      // lane group
  const int c = lane % 32;      // query column of this lane
  const uint32_t h = blockIdx.y;
  const uint32_t nqt = gridDim.x;
  const uint32_t qt = nqt - 1u - blockIdx.x;  // heaviest query tiles first
  const uint32_t L = a.L, Lq = a.Lq;
  const uint32_t off = L - Lq;                 // position of query 0

  const uint32_t q = qt * kPfQueriesPerBlock + wave * kPfQueriesPerWave + c;
  const bool q_live = q < Lq;
  const uint32_t qpos = q_live ? off + q : L - 1u;  // last key this query sees
  // keys this block needs: up to the last live query's position
  uint32_t qlast = qt * kPfQueriesPerBlock + kPfQueriesPerBlock - 1u;
  if (qlast >= Lq) qlast = Lq - 1u;
  const uint32_t kend = a.causal ? off + qlast + 1u : L;
  const uint32_t ntiles = (kend + kPfTileKeys - 1) / kPfTileKeys;
  // keys this wave needs (waves above the diagonal skip tiles)
  uint32_t wq_last = qt * kPfQueriesPerBlock + wave * kPfQueriesPerWave + kPfQueriesPerWave - 1u;
  if (wq_last >= Lq) wq_last = Lq - 1u;
  const uint32_t wave_kend = a.causal ? off + wq_last + 1u : L;

  // ---- this lane's query, dims 16*s + 8*g .. +8 for s = 0..7
  half8 qreg[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    qreg[s] = q_live ? *reinterpret_cast<const half8*>(a.q + ((size_t)q * a.H + h) * kHeadDim +
                                                          16 * s + 8 * g)
                     : half8{};

  // ---- tile loader: thread t covers keys 4*(t/16) .. +4, dims 8*(t%16) .. +8
  const int lk = 4 * (tid / 16), ld = 8 * (tid % 16);
  half8 pk0, pk1, pk2, pk3, pv0, pv1, pv2, pv3;
#define AOAKV_PF_LOAD(R, K0)                                                         \
  {                                                                                  \
    const uint32_t key = (K0) + lk + R;                                              \
    if (key < L) {                                                                   \
      const uint32_t phys = (uint32_t)a.kv_indices[key / kPageSize];                 \
      const size_t e = elem_off(a.g, phys, 0, h, key % kPageSize) + ld;              \
      pk##R = *reinterpret_cast<const half8*>(a.kv + e);                             \
      pv##R = *reinterpret_cast<const half8*>(a.kv + e + a.g.kv);                    \
    } else {                                                                         \
      pk##R = half8{};                                                               \
      pv##R = half8{};                                                               \
    }                                                                                \
  }
#define AOAKV_PF_LOAD_TILE(K0) \
  AOAKV_PF_LOAD(0, K0) AOAKV_PF_LOAD(1, K0) AOAKV_PF_LOAD(2, K0) AOAKV_PF_LOAD(3, K0)

  floatx16 acc_o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc_o[t] = floatx16{};
  float m_run = -INFINITY, l_run = 0.f;
  const float scale = a.sm_scale * kLog2e;

  AOAKV_PF_LOAD_TILE(0u)
  for (uint32_t it = 0; it < ntiles; ++it) {
    const uint32_t k0 = it * kPfTileKeys;
    __syncthreads();  // every wave is done reading the previous tile
    *reinterpret_cast<half8*>(&sK[(lk + 0) * kKRow + ld]) = pk0;
    *reinterpret_cast<half8*>(&sK[(lk + 1) * kKRow + ld]) = pk1;
    *reinterpret_cast<half8*>(&sK[(lk + 2) * kKRow + ld]) = pk2;
    *reinterpret_cast<half8*>(&sK[(lk + 3) * kKRow + ld]) = pk3;
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // V transposed: 4 keys of dim ld+j
      const half4 col = {pv0[j], pv1[j], pv2[j], pv3[j]};
      *reinterpret_cast<half4*>(&sVt[(ld + j) * kVRow + lk]) = col;
    }
    __syncthreads();
    if (it + 1 < ntiles) AOAKV_PF_LOAD_TILE(k0 + kPfTileKeys)  // in flight during the MFMAs
    if (k0 >= wave_kend) continue;  // wave-uniform: tile entirely above this wave's queries

    // ---- S^T = K Q^T for two 32-key sub-tiles
    floatx16 acc_s[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      acc_s[ks] = floatx16{};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const half8 ka = *reinterpret_cast<const half8*>(&sK[(ks * 32 + c) * kKRow + 16 * s + 8 * g]);
        acc_s[ks] = mfma32(ka, qreg[s], acc_s[ks]);
      }
    }
    // ---- scale, causal / length mask, running max of this query
    float mt = -INFINITY;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t key = k0 + ks * 32 + crow(i, g);
        const bool ok = key < L && (!a.causal || key <= qpos);
        const float x = ok ? acc_s[ks][i] * scale : -INFINITY;
        acc_s[ks][i] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = m_new == -INFINITY ? 1.f : exp2f(m_run - m_new);
    float lt = 0.f;
    half8 pb[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = m_new == -INFINITY ? 0.f : exp2f(acc_s[ks][i] - m_new);
        lt += p;
        pb[ks][i / 8][i % 8] = (f16)p;
      }
    }
    lt += __shfl_xor(lt, 32);
    l_run = l_run * alpha + lt;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc_o[t][i] *= alpha;

    // ---- O^T += V^T P^T.  B element j of half hf of sub-tile ks is the
    // probability of key ks*32 + 8*(2*hf + j/4) + 4*g + j%4, so the A operand
    // (V^T) lane reads those keys for its dim: two runs of 4 keys.
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f16* vrow = &sVt[(t * 32 + c) * kVRow];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int kb = ks * 32 + 16 * hf + 4 * g;
          const half4 lo = *reinterpret_cast<const half4*>(vrow + kb);
          const half4 hi = *reinterpret_cast<const half4*>(vrow + kb + 8);
          const half8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          acc_o[t] = mfma32(va, pb[ks][hf], acc_o[t]);
        }
      }
    }
  }

  // ---- o = O / l: lane holds its query's dims t*32 + crow(i, g)
  if (!q_live) return;
  const float inv_l = 1.f / l_run;
  f16* orow = a.o + ((size_t)q * a.H + h) * kHeadDim;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int i0 = 0; i0 < 16; i0 += 4) {
      half4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (f16)(acc_o[t][i0 + r] * inv_l);
      *reinterpret_cast<half4*>(orow + t * 32 + crow(i0, g)) = v;
    }
  }
}
#undef AOAKV_PF_LOAD_TILE
#undef AOAKV_PF_LOAD

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t s) {
  const uint32_t nqt = (a.Lq + kPfQueriesPerBlock - 1) / kPfQueriesPerBlock;
  hipLaunchKernelGGL(prefill_kernel, dim3(nqt, a.H), dim3(kPfThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace aoakv
