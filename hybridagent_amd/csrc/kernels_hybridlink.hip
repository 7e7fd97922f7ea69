// HybridLink latent step (hybridlink.py:17-28) for gfx950:
//   R(h) = post_ln(h + proj2(GELU(proj1(pre_ln(h)))))
// with bf16 parameters, as four launches:
//   k_layer_norm        a = LN(h)                      (one workgroup per row)
//   k_linear_bf16<GELU> g = bf16(GELU(bf16(a W1^T + b1)))  (kernels_linear_bf16.hip)
//   k_linear_bf16<RES>  r = bf16(h + bf16(g W2^T + b2))
//   k_layer_norm        out = LN(r)
// a and g are held in the linears' fragment order (linear_bf16.hpp): the
// first LayerNorm writes a that way, the GELU linear writes g that way.
// The rounding points are those of the torch bf16 module: every Linear,
// GELU, the residual add and each LayerNorm round to bf16 once.  At batch 32
// and H = 2816 each linear launch moves 15.9 MB of weights.
#include "common.hpp"
#include "launch.hpp"
#include "linear_bf16.hpp"

namespace w4a16 {

namespace {

constexpr int kLnThreads = 256;
constexpr int kLnChunks = 4;  // H <= 256 * 8 * 4 = 8192 held in registers

// sum over the workgroup in a fixed order (wave sums, then waves in order)
__device__ __forceinline__ float block_sum(float v, float* part) {
  v = wave_sum_f32(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) part[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kLnThreads / 64; ++i) t += part[i];
  __syncthreads();
  return t;
}

}  // namespace

// nn.LayerNorm over rows of H (fp32 statistics, two passes: mean, then the
// mean of squared deviations), affine with bf16 weight / bias, bf16 out
// (FRAG: in the bf16 linears' fragment order, rows padded to 16).
template <bool FRAG>
__global__ __launch_bounds__(kLnThreads) void k_layer_norm(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ b,
                                                          uint16_t* __restrict__ y, int H,
                                                          float eps) {
  __shared__ float part[kLnThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * H;
  const int n8 = H >> 3;
  float v[kLnChunks][8];
  float s = 0.f;
  // the row, then the affine parameters, all loads issued before the first
  // is used: one memory round trip, and the statistics wait only for the
  // row (loads complete in order)
  u32x4_t xv[kLnChunks], wv[kLnChunks], bv[kLnChunks];
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const int c8 = threadIdx.x + kLnThreads * q;
    xv[q] = c8 < n8 ? ld16(xr + 8 * c8) : u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const int c8 = min(threadIdx.x + kLnThreads * q, n8 - 1);
    wv[q] = ld16(w + 8 * c8);
    bv[q] = ld16(b + 8 * c8);
  }
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const u32x4_t u = xv[q];
    const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      v[q][2 * t] = bf16_bits_to_f32(w4[t] & 0xFFFFu);
      v[q][2 * t + 1] = bf16_bits_to_f32(w4[t] >> 16);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[q][e];
  }
  const float mean = block_sum(s, part) / (float)H;
  float d2 = 0.f;
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const int c8 = threadIdx.x + kLnThreads * q;
    if (c8 < n8) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[q][e] - mean;
        d2 = __builtin_fmaf(d, d, d2);
      }
    }
  }
  const float rstd = 1.0f / sqrtf(block_sum(d2, part) / (float)H + eps);
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const int c8 = threadIdx.x + kLnThreads * q;
    if (c8 < n8) {
      const uint32_t ww[4] = {wv[q].x, wv[q].y, wv[q].z, wv[q].w};
      const uint32_t bw[4] = {bv[q].x, bv[q].y, bv[q].z, bv[q].w};
      uint32_t o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float y0 = (v[q][2 * t] - mean) * rstd * bf16_bits_to_f32(ww[t] & 0xFFFFu) +
                         bf16_bits_to_f32(bw[t] & 0xFFFFu);
        const float y1 = (v[q][2 * t + 1] - mean) * rstd * bf16_bits_to_f32(ww[t] >> 16) +
                         bf16_bits_to_f32(bw[t] >> 16);
        o[t] = pack_bf16x2(y0, y1);
      }
      st16(y + (FRAG ? frag_index(row, 8 * c8, H) : row * H + 8 * c8), u32x4_t{o[0], o[1], o[2], o[3]});
    }
  }
}

hipError_t launch_layer_norm(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                             int64_t M, int H, float eps, bool frag, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (H % 8 != 0 || H > kLnThreads * 8 * kLnChunks || (frag && H % 32 != 0)) return hipErrorInvalidValue;
  if (frag)
    hipLaunchKernelGGL(k_layer_norm<true>, dim3((unsigned)M), dim3(kLnThreads), 0, s, x, w, b, y, H, eps);
  else
    hipLaunchKernelGGL(k_layer_norm<false>, dim3((unsigned)M), dim3(kLnThreads), 0, s, x, w, b, y, H, eps);
  return hipGetLastError();
}

}  // namespace w4a16
