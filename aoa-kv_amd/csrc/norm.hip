// RMSNorm of fp16 rows (gfx950): the reference's rms_norm_forward
// (kernels/aoa_kv/quest/ops/csrc/rms_norm.cu:76-150, called from
// quest/utils/__init__.py:54-67 and quest/models/llama.py:72):
//   out[i] = fp16( (x[i] * r) * w[i] ),  r = 1 / sqrt(sum_j x[j]^2 / n + eps)
// with x, w widened to fp32, the products in that order and one rounding.
//
// One workgroup of 256 threads per row.  Thread t owns the 16-byte vectors
// t, t + 256, ... of its row and keeps up to kNormVecs of them in registers
// between the two passes (rows up to 256 * 8 * kNormVecs = 16384 elements);
// longer rows read their vectors again for the second pass.  The sum of
// squares is an fp32 sum per thread, then a DPP row sum, the four rows of a
// wave and the four waves in LDS.
#include "kernels.hpp"

namespace aoakv {

constexpr int kNormThreads = 256;
constexpr int kNormVecs = 8;

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(RmsNormArgs a) {
  __shared__ float s_part[kNormThreads / kWave];
  const uint32_t tid = threadIdx.x;
  const uint32_t nvec = a.n / (uint32_t)kVec;
  const f16* x = a.x + (size_t)blockIdx.x * a.n;
  f16* out = a.out + (size_t)blockIdx.x * a.n;

  H8 xv[kNormVecs];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormVecs; ++i) {
    const uint32_t v = tid + (uint32_t)i * kNormThreads;
    xv[i] = ld16(x + (size_t)(v < nvec ? v : 0u) * kVec);
  }
#pragma unroll
  for (int i = 0; i < kNormVecs; ++i) {
    if (tid + (uint32_t)i * kNormThreads < nvec) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float f = (float)xv[i].v[j];
        ss = ss + f * f;
      }
    }
  }
  for (uint32_t v = tid + kNormVecs * kNormThreads; v < nvec; v += kNormThreads) {
    const H8 t = ld16(x + (size_t)v * kVec);
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const float f = (float)t.v[j];
      ss = ss + f * f;
    }
  }
  ss = cross_row_sum(row_sum16(ss));
  if (__lane_id() == 0u) s_part[tid / kWave] = ss;
  __syncthreads();
  const float total = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  const float r = 1.0f / sqrtf(total / (float)a.n + a.eps);

  auto norm8 = [&](const H8& xx, uint32_t v) {
    const H8 w = ld16(a.w + (size_t)v * kVec);
    H8 o;
#pragma unroll
    for (int j = 0; j < kVec; ++j) o.v[j] = r16(((float)xx.v[j] * r) * (float)w.v[j]);
    st16(out + (size_t)v * kVec, o);
  };
#pragma unroll
  for (int i = 0; i < kNormVecs; ++i) {
    const uint32_t v = tid + (uint32_t)i * kNormThreads;
    if (v < nvec) norm8(xv[i], v);
  }
  for (uint32_t v = tid + kNormVecs * kNormThreads; v < nvec; v += kNormThreads)
    norm8(ld16(x + (size_t)v * kVec), v);
}

hipError_t launch_rms_norm(const RmsNormArgs& a, uint32_t rows, hipStream_t s) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kNormThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace aoakv
