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

// The weighted top-k combine of one token row (k_combine's arithmetic:
// bf16(sum_j bf16(bf16(w[t, j]) * dn[t*k + j]))), the residual add and the
// RMSNorm of the sum (k_add_rms_norm's arithmetic and reduction order) in
// one workgroup per row -- the latent harness's h <- h + MoE(...) followed
// by the next layer's norm, without the combine's output round trip:
//   out = combine(...)[t], h_out = bf16(h + out), y = bf16((h_out * r) * w)
// topk <= 8; every load of the row (its k down-projection pieces, h and
// the norm weight) is issued before the first is used.
__global__ __launch_bounds__(kNormThreads) void k_combine_add_rms_norm(
    const uint16_t* __restrict__ dn, const int64_t* __restrict__ idx, const float* __restrict__ tw,
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
    uint16_t* __restrict__ h_out, uint16_t* __restrict__ y, int topk, int E, int H, float eps) {
  constexpr int KMAX = 8;
  __shared__ float s_part[kNormThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int n8 = H >> 3;
  const int64_t r0 = row * topk;
  int64_t ex[KMAX];
  float wv[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const int64_t r = r0 + (j < topk ? j : 0);
    ex[j] = idx[r];
    wv[j] = tw[r];
  }
  u32x4_t d[kNormChunks][KMAX], hv[kNormChunks], gv[kNormChunks];
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = min(tid + kNormThreads * q, n8 - 1);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) d[q][j] = ld16(dn + (r0 + (j < topk ? j : 0)) * H + 8 * c8);
    hv[q] = ld16(h + row * H + 8 * c8);
    gv[q] = ld16(w + 8 * c8);
  }
  float ss = 0.f;
  u32x4_t xv[kNormChunks];
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = tid + kNormThreads * q;
    xv[q] = u32x4_t{0u, 0u, 0u, 0u};
    if (c8 >= n8) continue;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < topk && ex[j] >= 0 && ex[j] < E) {
        const float wb = round_bf16(wv[j]);
        const uint32_t dw[4] = {d[q][j].x, d[q][j].y, d[q][j].z, d[q][j].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          acc[2 * t] += round_bf16(bf16_bits_to_f32(dw[t] & 0xFFFFu) * wb);
          acc[2 * t + 1] += round_bf16(bf16_bits_to_f32(dw[t] >> 16) * wb);
        }
      }
    }
    const uint32_t o4[4] = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                            pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7])};
    if (out != nullptr) st16(out + row * H + 8 * c8, u32x4_t{o4[0], o4[1], o4[2], o4[3]});
    const uint32_t h4[4] = {hv[q].x, hv[q].y, hv[q].z, hv[q].w};
    uint32_t x4[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float v[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float a = bf16_bits_to_f32(hh ? (h4[t] >> 16) : (h4[t] & 0xFFFFu));
        const float b = bf16_bits_to_f32(hh ? (o4[t] >> 16) : (o4[t] & 0xFFFFu));
        v[hh] = round_bf16(a + b);
        ss = __builtin_fmaf(v[hh], v[hh], ss);
      }
      x4[t] = pack_bf16x2(v[0], v[1]);
    }
    xv[q] = u32x4_t{x4[0], x4[1], x4[2], x4[3]};
    st16(h_out + row * H + 8 * c8, xv[q]);
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
    const uint32_t x4[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
    const uint32_t w4[4] = {gv[q].x, gv[q].y, gv[q].z, gv[q].w};
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

hipError_t launch_combine_add_rms_norm(const uint16_t* dn, const int64_t* idx, const float* tw, const uint16_t* h,
                                       const uint16_t* w, uint16_t* out, uint16_t* h_out, uint16_t* y, int64_t M,
                                       int topk, int E, int H, float eps, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (topk <= 0 || topk > 8 || H % 8 != 0 || H > kNormThreads * kNormChunks * 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_combine_add_rms_norm, dim3((unsigned)M), dim3(kNormThreads), 0, s, dn, idx, tw, h, w, out,
                     h_out, y, topk, E, H, eps);
  return hipGetLastError();
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
