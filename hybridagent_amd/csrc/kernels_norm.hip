// Residual add + RMSNorm of the latent harness's MoE input
// (TF:models/gemma4/modeling_gemma4.py:197-215 -- fp32 x * rsqrt(mean(x^2) +
// eps) * w, back to the input dtype -- and the harness's h <- h + MoE(...)):
//   x = bf16(h + delta)                       (h_out; with delta null x = h)
//   y = bf16((x * rsqrt(mean(x^2) + eps)) * w)  in fp32, in that order
// One 256-thread workgroup per row; the sum of squares in a fixed order
// (each thread over its chunks, then wavefront sums, then the four
// wavefronts in order).
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // 16-byte chunks per thread: H <= 256 * 4 * 8

__global__ __launch_bounds__(kNormThreads) void k_add_rms_norm(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ delta,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ h_out, uint16_t* __restrict__ y,
    int H, float eps) {
  __shared__ float s_part[kNormThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int n8 = H >> 3;
  const uint16_t* hr = h + row * H;
  const uint16_t* dr = delta != nullptr ? delta + row * H : nullptr;
  u32x4_t xv[kNormChunks], dv[kNormChunks];
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = tid + kNormThreads * q;
    xv[q] = u32x4_t{0u, 0u, 0u, 0u};
    dv[q] = u32x4_t{0u, 0u, 0u, 0u};
    if (c8 < n8) {
      xv[q] = ld16(hr + 8 * c8);
      if (dr != nullptr) dv[q] = ld16(dr + 8 * c8);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = tid + kNormThreads * q;
    if (c8 >= n8) continue;
    const uint32_t x4[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
    const uint32_t d4[4] = {dv[q].x, dv[q].y, dv[q].z, dv[q].w};
    uint32_t o4[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float v[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float a = bf16_bits_to_f32(hh ? (x4[t] >> 16) : (x4[t] & 0xFFFFu));
        const float b = bf16_bits_to_f32(hh ? (d4[t] >> 16) : (d4[t] & 0xFFFFu));
        v[hh] = dr != nullptr ? round_bf16(a + b) : a;
        ss = __builtin_fmaf(v[hh], v[hh], ss);
      }
      o4[t] = pack_bf16x2(v[0], v[1]);
    }
    xv[q] = u32x4_t{o4[0], o4[1], o4[2], o4[3]};
    if (dr != nullptr && h_out != nullptr) st16(h_out + row * H + 8 * c8, xv[q]);
  }
  ss = wave_sum_f32(ss);
  if (lane == 0) s_part[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
  const float r = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = tid + kNormThreads * q;
    if (c8 >= n8) continue;
    const u32x4_t wv = ld16(w + 8 * c8);
    const uint32_t x4[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
    const uint32_t w4[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t o4[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float v[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float x = bf16_bits_to_f32(hh ? (x4[t] >> 16) : (x4[t] & 0xFFFFu));
        const float g = bf16_bits_to_f32(hh ? (w4[t] >> 16) : (w4[t] & 0xFFFFu));
        v[hh] = (x * r) * g;
      }
      o4[t] = pack_bf16x2(v[0], v[1]);
    }
    st16(y + row * H + 8 * c8, u32x4_t{o4[0], o4[1], o4[2], o4[3]});
  }
}

hipError_t launch_add_rms_norm(const uint16_t* h, const uint16_t* delta, const uint16_t* w,
                               uint16_t* h_out, uint16_t* y, int64_t M, int H, float eps,
                               hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (H % 8 != 0 || H > kNormThreads * kNormChunks * 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_add_rms_norm, dim3((unsigned)M), dim3(kNormThreads), 0, s, h, delta, w,
                     h_out, y, H, eps);
  return hipGetLastError();
}

}  // namespace w4a16
