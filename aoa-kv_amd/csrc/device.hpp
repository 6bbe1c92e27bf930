// Device-side helpers shared by the libaoakv kernels (gfx950 / CDNA4).
//
// Wave = 64 lanes.  A 128-dim fp16 row is 256 B = 16 lanes x 16 B, so most
// kernels view a wave as four 16-lane "rows" (the DPP row of the hardware),
// each row owning one (page or token, head) vector: lane l holds dims
// [8*(l%16), 8*(l%16)+8).  Reductions inside a row use DPP; across rows a
// wave shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aoakv {

using f16 = _Float16;

constexpr int kWave = 64;
constexpr int kHeadDim = 128;
constexpr int kPageSize = 16;
constexpr int kLanesPerRow = 16;   // lanes covering one 128-dim fp16 vector
constexpr int kVec = 8;            // fp16 elements per lane per vector

// sqrt(128) rounded to fp32: the simulation divides by math.sqrt(head_dim)
// as an fp32 true division (filter_util.py:329, quest_attention.py:268).
constexpr float kSqrtHeadDim = 11.313708498984761f;
constexpr float kRcpSqrtHeadDim = 1.0f / kSqrtHeadDim;  // fp32(1 / fp32(sqrt(128)))

struct alignas(16) H8 {
  f16 v[8];
};

// ---------------------------------------------------------------- layout

// Element strides inside one page of a paged cache.
struct PageGeom {
  uint32_t page, kv, head, tok;
};

__host__ __device__ inline PageGeom make_geom(uint32_t layout, uint32_t H, uint32_t S,
                                              uint32_t D) {
  PageGeom g;
  g.page = 2u * S * H * D;
  g.kv = S * H * D;
  if (layout == 0u) {  // NHD: [2][S][H][D]
    g.tok = H * D;
    g.head = D;
  } else {  // HND: [2][H][S][D]
    g.head = S * D;
    g.tok = D;
  }
  return g;
}

__device__ inline size_t elem_off(const PageGeom& g, uint32_t page, uint32_t kv, uint32_t head,
                                  uint32_t tok) {
  return (size_t)page * g.page + (size_t)kv * g.kv + (size_t)head * g.head +
         (size_t)tok * g.tok;
}

// ---------------------------------------------------------------- loads/stores

__device__ inline H8 ld16(const f16* p) {
  uint4 u = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(H8, u);
}
// 16 bytes of data read once per launch (the K/V gather, the scoring's
// metadata) with a non-temporal load: on an MI355X, 256 workgroups gathering
// 64 KB each of random 4 KB blocks took 1.16 us at the median and 2.8 at
// the slowest this way, against 2.6 and 6.0 us with plain loads
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ inline H8 ld16_nt(const f16* p) {
  return __builtin_bit_cast(H8, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}
__device__ inline void st16(f16* p, const H8& x) {
  *reinterpret_cast<uint4*>(p) = __builtin_bit_cast(uint4, x);
}
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// x / sqrt(128) in fp32, correctly rounded for every fp16 value x: the
// reciprocal product plus one Newton correction gives the rounded quotient
// for all finite fp16 inputs (exhaustive check in tests/test_oracle.py) but
// the sign of a zero, which copysign restores; inf and NaN take the product.
// Three VALU operations where the IEEE division sequence takes about ten.
__device__ inline float div_sqrt_head_dim_f16(float x) {
  const float q0 = x * kRcpSqrtHeadDim;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, kSqrtHeadDim, x), kRcpSqrtHeadDim, q0);
  return __builtin_isfinite(x) ? __builtin_copysignf(q1, x) : q0;
}
// elements 2m, 2m+1 of x (one 32-bit register)
__device__ inline half2v half_pair(const H8& x, int m) { return half2v{x.v[2 * m], x.v[2 * m + 1]}; }

// ---------------------------------------------------------------- DPP / shuffles

template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// DPP controls: quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror.
constexpr int kQuadSwap1 = 0xB1;
constexpr int kQuadSwap2 = 0x4E;
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowShl1 = 0x101;  // row_shl:1 (lane l of a row reads lane l + 1)

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ inline float row_sum16(float x) {
  x = x + dpp<kQuadSwap1>(x);
  x = x + dpp<kQuadSwap2>(x);
  x = x + dpp<kRowHalfMirror>(x);
  x = x + dpp<kRowMirror>(x);
  return x;
}

__device__ inline float row_max16(float x) {
  x = fmaxf(x, dpp<kQuadSwap1>(x));
  x = fmaxf(x, dpp<kQuadSwap2>(x));
  x = fmaxf(x, dpp<kRowHalfMirror>(x));
  x = fmaxf(x, dpp<kRowMirror>(x));
  return x;
}

// Across the four rows of a wave (lanes l, l^16, l^32, l^48).
__device__ inline float cross_row_sum(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}
__device__ inline float cross_row_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

// ---------------------------------------------------------------- fp16 arithmetic
// The reference simulation runs fp16 tensors through torch's CPU kernels:
// every elementwise op is computed in fp32 and rounded once to fp16 (RNE).
// These helpers reproduce that; the library is compiled with
// -ffp-contract=off so no multiply-add is fused across a rounding point.

__device__ inline f16 r16(float x) { return (f16)x; }

// update_mean_filter (filter_util.py:669-679): (m*n + v)/(n+1), each of the
// three fp16 ops rounded to fp16.  n is the number of tokens already in the
// page.
__device__ inline f16 running_mean(f16 m, f16 v, uint32_t n) {
  f16 t = r16((float)m * (float)n);
  t = r16((float)t + (float)v);
  return r16((float)t / (float)(n + 1u));
}

// log(norm(V̄) + 1e-8) of one 128-dim fp16 vector held by a 16-lane row
// (8 dims per lane, lane order = dim order), as torch computes it on fp16
// (filter_util.py:325):
//   norm: fp32 sum of squares in dim order 0..127, sqrtf, round to fp16;
//   + 1e-8: fp16 op (leaves every fp16 value unchanged; kept for clarity);
//   log: correctly rounded fp32 log (via fp64), rounded to fp16.
// The sequential fp32 chain is carried lane to lane across the row.
// Returns the fp16 log-norm in every lane of the row.
__device__ inline f16 log_norm_row(const H8& vbar, uint32_t lane16) {
  float acc = 0.f;
#pragma unroll
  for (int src = 0; src < kLanesPerRow; ++src) {
    if ((int)lane16 == src) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        float x = (float)vbar.v[j];
        float sq = x * x;
        acc = acc + sq;
      }
    }
    // hand the running sum to the next lane of the row
    acc = __shfl(acc, (int)((__lane_id() & ~15u) | (uint32_t)src), kWave);
  }
  // the correctly rounded fp32 root (torch's sqrtf): the fp64 root rounded
  // once to fp32 is exactly that (53 >= 2 * 24 + 2 bits).  __fsqrt_rn is not
  // used: this toolchain's header maps it to the native approximation, whose
  // last bit can differ, and an fp32 root on an fp16 midpoint then rounds to
  // the other fp16 neighbour (seen at one page-head of 65,536 at config 3a).
  f16 nrm = r16((float)__builtin_sqrt((double)acc));
  nrm = r16((float)nrm + 1e-8f);
  double ln = log((double)(float)nrm);
  return r16((float)ln);
}

// ---------------------------------------------------------------- RoPE
// Llama rotary embedding in the rotate-half form (QKApplyRotaryInPlaceKernel,
// decode_page.cuh:785-840, which the reference tests against HF's
// apply_rotary_pos_emb, quest/tests/test_rope.py:17-30).  For dim d of a
// 128-dim vector at position pos, with i = d mod 64:
//   f_i = rcp_scale * rcp_theta^(i / 64),   a = fp32(pos) * f_i,
//   out_d = x_d cos a - x_{d+64} sin a   (d < 64)
//   out_d = x_d cos a + x_{d-64} sin a   (d >= 64),
// with f_i evaluated in fp64 and rounded to fp32 (so it is the correctly
// rounded frequency: at position 10^4 one ulp of f_i moves the angle by
// ~10^-3; the host computes the 64 of them once per launch, rope_freqs), the
// angle and rotation in fp32 with the accurate sincosf, and one rounding to
// fp16 at the end.  Lane l16
// of a 16-lane row holds dims 8*l16 .. 8*l16 + 7, so the partner dims d +- 64
// are in lane l16 ^ 8 of the same row (DPP row_ror:8).
struct RopeTable {
  float c[kVec], s[kVec];  // cos / sin of this lane's 8 dims at one position
};

// freqs: the 64 frequencies f_i (kernel argument)
__device__ inline RopeTable rope_table(uint32_t pos, uint32_t l16, const float* freqs) {
  RopeTable t;
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const uint32_t i = (l16 * kVec + (uint32_t)j) % (kHeadDim / 2);
    sincosf((float)pos * freqs[i], &t.s[j], &t.c[j]);
  }
  return t;
}

__device__ inline H8 rope_row(const H8& x, const RopeTable& t, uint32_t l16) {
  const uint4 u = __builtin_bit_cast(uint4, x);
  uint4 pu;  // the partner lane's 8 dims
  pu.x = (uint32_t)__builtin_amdgcn_mov_dpp((int)u.x, 0x128, 0xF, 0xF, false);  // row_ror:8
  pu.y = (uint32_t)__builtin_amdgcn_mov_dpp((int)u.y, 0x128, 0xF, 0xF, false);
  pu.z = (uint32_t)__builtin_amdgcn_mov_dpp((int)u.z, 0x128, 0xF, 0xF, false);
  pu.w = (uint32_t)__builtin_amdgcn_mov_dpp((int)u.w, 0x128, 0xF, 0xF, false);
  const H8 p = __builtin_bit_cast(H8, pu);
  const bool low = l16 < 8u;  // dims < 64: the partner term enters negated
  H8 y;
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const float a = (float)x.v[j] * t.c[j];
    const float b = (float)p.v[j] * t.s[j];
    y.v[j] = r16(low ? a - b : a + b);
  }
  return y;
}

// ---------------------------------------------------------------- cross-workgroup handoff
// gfx950 has one L2 per XCD and the L2s are not coherent with each other.
// An agent-scope __threadfence() therefore writes back and invalidates the
// whole L2 -- far too slow to run in every workgroup.  Data handed from one
// workgroup to another instead travels through agent-coherent accesses
// (relaxed agent-scope atomic loads / stores, `sc1`), which go to the
// memory-side coherence point, and the handoff is ordered by waiting for the
// stores to complete before the arrival counter is incremented (RMW atomics
// are performed at the coherence point).

__device__ inline void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent_i32(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld_agent_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every workgroup of a group of n calls this once after its st_agent()
// stores; it returns true (in all threads) in the workgroup that arrives
// last, which may then ld_agent() everything the others stored.  The last
// workgroup resets the counter to zero for the next launch.
__device__ inline bool arrive_last(uint32_t* counter, uint32_t n, uint32_t* s_flag) {
  // the vector-memory counter reaches zero only when this wave's stores are
  // complete; the "memory" clobber keeps the compiler from moving them
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = prev == n - 1u ? 1u : 0u;
    if (prev == n - 1u) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return *s_flag != 0u;
}

// Map an fp32 score to a uint32 key with the same order (larger float ->
// larger key).  -0.0 and +0.0 map to adjacent keys (torch.topk treats them
// as equal; scores of exactly zero with both signs do not arise).
__device__ inline uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Selection flags (the bits of the C ABI's AOAKV_FLAG_*).
constexpr uint32_t kFlagValueAware = 1u;
constexpr uint32_t kFlagFixed = 2u;
constexpr uint32_t kFlagQuestKernel = 8u;

// Pages attended per (sequence, kv head).
//   simulation:   k = min(max(3, min(L, budget) / page_size), P)
//                 (filter_util.py:373, quest_attention.py:326)
//   quest_kernel: k = min(max(1, budget / page_size), P): the last page plus
//                 k - 1 pages selected from the others (controller.py:118,
//                 quest/utils/__init__.py:237)
__host__ __device__ inline uint32_t num_selected_pages(uint32_t L, uint32_t budget,
                                                       uint32_t page_size, uint32_t P,
                                                       uint32_t flags) {
  uint32_t k;
  if (flags & kFlagQuestKernel) {
    k = budget / page_size;
    if (k < 1u) k = 1u;
  } else {
    const uint32_t tb = L < budget ? L : budget;
    k = tb / page_size;
    if (k < 3u) k = 3u;
  }
  return k < P ? k : P;
}

}  // namespace aoakv
