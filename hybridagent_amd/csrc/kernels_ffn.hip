// Row kernels of the post-attention FFN block _ffn_moe_4bit_step
// (backends.py:101-126), around the shared-MLP linears
// (kernels_linear_bf16.hip) and the MoE layer:
//
//   k_ffn_pre   h      = rms_norm(attn_out) * post_attn_ln_w        (:102)
//               res    = bf16(residual + h)                         (:103)
//               h_ff   = rms_norm(res) * pre_ff_ln_w                (:105)
//               h2_in  = rms_norm(res) * pre_ff_ln2_w               (:119)
//   k_ffn_post  h_1    = rms_norm(h_mlp) * post_ff_ln1_w            (:109)
//               h_2    = rms_norm(moe_out) * post_ff_ln2_w          (:123)
//               h_comb = rms_norm(bf16(h_1 + h_2)) * post_ff_ln_w   (:125)
//               out    = bf16(bf16(res + h_comb) * layer_scalar)    (:126)
//
// rms_norm(x) * w is F.rms_norm on bf16 rows: fp32 x * rsqrt(mean(x^2) + eps),
// times w, rounded to bf16 (each norm's output is a bf16 tensor).  One
// 256-thread workgroup per row; every sum of squares is taken in a fixed
// order (each thread over its chunks, wavefront sums, the four wavefronts in
// order), so a row's result does not depend on the batch around it.
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kFfnThreads = 256;
constexpr int kFfnChunks = 4;  // 16-byte chunks per thread: H <= 256 * 4 * 8

// sums of two values over the workgroup in a fixed order
__device__ __forceinline__ float2 block_sum2(float a, float b, float2* part) {
  a = wave_sum_f32(a);
  b = wave_sum_f32(b);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) part[w] = make_float2(a, b);
  __syncthreads();
  float2 t = part[0];
#pragma unroll
  for (int i = 1; i < kFfnThreads / 64; ++i) {
    t.x += part[i].x;
    t.y += part[i].y;
  }
  __syncthreads();
  return t;
}

// a row's chunk q of this thread (8 bf16 values) as floats; zero past H
struct Row8 {
  float v[8];
};

__device__ __forceinline__ Row8 load8(const uint16_t* row, int c8, bool ok) {
  Row8 r;
  const u32x4_t u = ok ? ld16(row + 8 * c8) : u32x4_t{0u, 0u, 0u, 0u};
  const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    r.v[2 * t] = bf16_bits_to_f32(w4[t] & 0xFFFFu);
    r.v[2 * t + 1] = bf16_bits_to_f32(w4[t] >> 16);
  }
  return r;
}

// the 16-byte chunk itself, converted only where used (a conversion right
// after the load would wait for it)
__device__ __forceinline__ u32x4_t raw8(const uint16_t* row, int c8, bool ok) {
  return ok ? ld16(row + 8 * c8) : u32x4_t{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ Row8 conv8(const u32x4_t& u) {
  Row8 r;
  const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    r.v[2 * t] = bf16_bits_to_f32(w4[t] & 0xFFFFu);
    r.v[2 * t + 1] = bf16_bits_to_f32(w4[t] >> 16);
  }
  return r;
}

__device__ __forceinline__ void store8(uint16_t* row, int c8, const float* v) {
  st16(row + 8 * c8, u32x4_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                             pack_bf16x2(v[6], v[7])});
}

__device__ __forceinline__ float sumsq8(const Row8& r) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = __builtin_fmaf(r.v[e], r.v[e], s);
  return s;
}

// bf16((x * rstd) * w) for the 8 values of a chunk, as floats
__device__ __forceinline__ void norm8(const Row8& x, float rstd, const Row8& w, float* out) {
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = round_bf16((x.v[e] * rstd) * w.v[e]);
}

}  // namespace

__global__ __launch_bounds__(kFfnThreads) void k_ffn_pre(
    const uint16_t* __restrict__ attn, const uint16_t* __restrict__ res, const uint16_t* __restrict__ w_pa,
    const uint16_t* __restrict__ w_pf, const uint16_t* __restrict__ w_pf2, uint16_t* __restrict__ res_out,
    uint16_t* __restrict__ h_ff, uint16_t* __restrict__ h2_in, int H, float eps) {
  __shared__ float2 part[kFfnThreads / 64];
  const int64_t off = (int64_t)blockIdx.x * H;
  const int n8 = H >> 3;
  Row8 a[kFfnChunks], r[kFfnChunks];
  // every load issued before the first reduction: the rows, then the three
  // norms' weights (one memory round trip instead of three)
  u32x4_t wa[kFfnChunks], wf[kFfnChunks], wf2[kFfnChunks];
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    a[q] = load8(attn + off, c8, c8 < n8);
    r[q] = load8(res + off, c8, c8 < n8);
  }
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    wa[q] = raw8(w_pa, c8, c8 < n8);
    wf[q] = raw8(w_pf, c8, c8 < n8);
    wf2[q] = raw8(w_pf2, c8, c8 < n8);
  }
  float ssa = 0.f;
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) ssa += sumsq8(a[q]);
  const float rsa = 1.0f / sqrtf(block_sum2(ssa, 0.f, part).x / (float)H + eps);
  float ssr = 0.f;
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    const bool ok = c8 < n8;
    const Row8 w = conv8(wa[q]);
    float h[8];
    norm8(a[q], rsa, w, h);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[q].v[e] = ok ? round_bf16(r[q].v[e] + h[e]) : 0.f;
    if (ok) store8(res_out + off, c8, r[q].v);
    ssr += sumsq8(r[q]);
  }
  const float rsr = 1.0f / sqrtf(block_sum2(ssr, 0.f, part).x / (float)H + eps);
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    if (c8 >= n8) continue;
    float o[8];
    norm8(r[q], rsr, conv8(wf[q]), o);
    store8(h_ff + off, c8, o);
    norm8(r[q], rsr, conv8(wf2[q]), o);
    store8(h2_in + off, c8, o);
  }
}

__global__ __launch_bounds__(kFfnThreads) void k_ffn_post(
    const uint16_t* __restrict__ mlp, const uint16_t* __restrict__ moe, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ w1, const uint16_t* __restrict__ w2, const uint16_t* __restrict__ w3,
    const uint16_t* __restrict__ layer_scalar, uint16_t* __restrict__ out, int H, float eps) {
  __shared__ float2 part[kFfnThreads / 64];
  const int64_t off = (int64_t)blockIdx.x * H;
  const int n8 = H >> 3;
  Row8 m[kFfnChunks], e2[kFfnChunks];
  // every load issued before the first reduction: the two rows, then the
  // three norms' weights and the residual row (one memory round trip)
  u32x4_t w1r[kFfnChunks], w2r[kFfnChunks], w3r[kFfnChunks], rr[kFfnChunks];
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    m[q] = load8(mlp + off, c8, c8 < n8);
    e2[q] = load8(moe + off, c8, c8 < n8);
  }
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    w1r[q] = raw8(w1, c8, c8 < n8);
    w2r[q] = raw8(w2, c8, c8 < n8);
    w3r[q] = raw8(w3, c8, c8 < n8);
    rr[q] = raw8(res + off, c8, c8 < n8);
  }
  const float ls = bf16_bits_to_f32(layer_scalar[0]);
  float ssm = 0.f, sse = 0.f;
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    ssm += sumsq8(m[q]);
    sse += sumsq8(e2[q]);
  }
  const float2 ss = block_sum2(ssm, sse, part);
  const float rm = 1.0f / sqrtf(ss.x / (float)H + eps);
  const float re = 1.0f / sqrtf(ss.y / (float)H + eps);
  // c = bf16(h_1 + h_2), kept in m[]
  float ssc = 0.f;
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    const bool ok = c8 < n8;
    float h1[8], h2[8];
    norm8(m[q], rm, conv8(w1r[q]), h1);
    norm8(e2[q], re, conv8(w2r[q]), h2);
#pragma unroll
    for (int e = 0; e < 8; ++e) m[q].v[e] = ok ? round_bf16(h1[e] + h2[e]) : 0.f;
    ssc += sumsq8(m[q]);
  }
  const float rc = 1.0f / sqrtf(block_sum2(ssc, 0.f, part).x / (float)H + eps);
#pragma unroll
  for (int q = 0; q < kFfnChunks; ++q) {
    const int c8 = threadIdx.x + kFfnThreads * q;
    if (c8 >= n8) continue;
    float hc[8];
    norm8(m[q], rc, conv8(w3r[q]), hc);
    const Row8 r = conv8(rr[q]);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = round_bf16(r.v[e] + hc[e]) * ls;
    store8(out + off, c8, o);
  }
}

hipError_t launch_ffn_pre(const uint16_t* attn, const uint16_t* res, const uint16_t* w_pa,
                          const uint16_t* w_pf, const uint16_t* w_pf2, uint16_t* res_out, uint16_t* h_ff,
                          uint16_t* h2_in, int64_t M, int H, float eps, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (H % 8 != 0 || H > kFfnThreads * kFfnChunks * 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ffn_pre, dim3((unsigned)M), dim3(kFfnThreads), 0, s, attn, res, w_pa, w_pf, w_pf2,
                     res_out, h_ff, h2_in, H, eps);
  return hipGetLastError();
}

hipError_t launch_ffn_post(const uint16_t* mlp, const uint16_t* moe, const uint16_t* res,
                           const uint16_t* w1, const uint16_t* w2, const uint16_t* w3,
                           const uint16_t* layer_scalar, uint16_t* out, int64_t M, int H, float eps,
                           hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (H % 8 != 0 || H > kFfnThreads * kFfnChunks * 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ffn_post, dim3((unsigned)M), dim3(kFfnThreads), 0, s, mlp, moe, res, w1, w2, w3,
                     layer_scalar, out, H, eps);
  return hipGetLastError();
}

}  // namespace w4a16
