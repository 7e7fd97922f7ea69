// HybridLink latent step (hybridlink.py:17-28) for gfx950:
//   R(h) = post_ln(h + proj2(GELU(proj1(pre_ln(h)))))
// with bf16 parameters, as four launches:
//   k_layer_norm        a = LN(h)                      (one workgroup per row)
//   k_linear_bf16<GELU> g = bf16(GELU(bf16(a W1^T + b1)))
//   k_linear_bf16<RES>  r = bf16(h + bf16(g W2^T + b2))
//   k_layer_norm        out = LN(r)
// The rounding points are those of the torch bf16 module: every Linear,
// GELU, the residual add and each LayerNorm round to bf16 once.
//
// k_linear_bf16 streams the weights once: a workgroup owns 16 output columns
// (one MFMA column tile) for up to 64 rows; its eight wavefronts split K and
// issue all their weight and activation loads before the first MFMA (11 + 11
// MT loads of 16 bytes per lane at K = 2816), then the eight partial tiles
// are summed in LDS in wavefront
// order (deterministic) and the epilogue applies bias, GELU or the residual.
// At batch 32 and H = 2816 a launch moves 15.9 MB of weights.
#include "common.hpp"
#include "launch.hpp"

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
// mean of squared deviations), affine with bf16 weight / bias, bf16 out.
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
  // the affine parameters are loaded with the row, so the row's statistics
  // and the parameters arrive in one memory round trip
  u32x4_t wv[kLnChunks], bv[kLnChunks];
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const int c8 = min(threadIdx.x + kLnThreads * q, n8 - 1);
    wv[q] = ld16(w + 8 * c8);
    bv[q] = ld16(b + 8 * c8);
  }
#pragma unroll
  for (int q = 0; q < kLnChunks; ++q) {
    const int c8 = threadIdx.x + kLnThreads * q;
    const u32x4_t u = c8 < n8 ? ld16(xr + 8 * c8) : u32x4_t{0u, 0u, 0u, 0u};
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
      st16(y + row * H + 8 * c8, u32x4_t{o[0], o[1], o[2], o[3]});
    }
  }
}

hipError_t launch_layer_norm(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                             int64_t M, int H, float eps, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (H % 8 != 0 || H > kLnThreads * 8 * kLnChunks) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_layer_norm, dim3((unsigned)M), dim3(kLnThreads), 0, s, x, w, b, y, H, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// out[m, n] = epilogue(sum_k x[m, k] W[n, k] + bias[n]) for M rows (MT m-tiles
// of 16 per workgroup, grid.y = ceil(M / 16 MT)), bf16 weights [N, K].
// ---------------------------------------------------------------------------
constexpr int kLinWaves = 8;
constexpr int kLinMaxSteps = 12;  // 32-wide k steps per wavefront held in registers

template <int MT, int EPI>
__global__ __launch_bounds__(64 * kLinWaves) void k_linear_bf16(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ res,
    uint16_t* __restrict__ out, int M, int N, int K, int steps_per_wave) {
  __shared__ f32x4_t red[kLinWaves][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * MT;
  const int nsteps = K >> 5;
  const int c0 = wave * steps_per_wave;
  const int c1 = min(nsteps, c0 + steps_per_wave);
  // this lane's weight row and activation rows (clamped: columns past N and
  // rows past M compute values that are not stored)
  const uint16_t* wrow = W + (int64_t)min(n0 + j, N - 1) * K + 8 * kb;
  const uint16_t* xrow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) xrow[i] = x + (int64_t)min(m0 + 16 * i + j, M - 1) * K + 8 * kb;
  f32x4_t acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // every load of the wavefront's k range before the first MFMA: the
  // weights (HBM), then the activation fragments (L2-resident), so the
  // wavefront waits for memory once.  Steps past the range load its last
  // step again (unused; a wavefront with an empty range loads the matrix's
  // last step), so every wavefront issues the same loads.
  auto step_at = [&](int c) { return min(max(c0, min(c0 + c, c1 - 1)), nsteps - 1); };
  u32x4_t wv[kLinMaxSteps];
#pragma unroll
  for (int c = 0; c < kLinMaxSteps; ++c) wv[c] = ld16(wrow + 32 * step_at(c));
  u32x4_t av[kLinMaxSteps][MT];
#pragma unroll
  for (int c = 0; c < kLinMaxSteps; ++c)
#pragma unroll
    for (int i = 0; i < MT; ++i) av[c][i] = ld16(xrow[i] + 32 * step_at(c));
#pragma unroll
  for (int c = 0; c < kLinMaxSteps; ++c) {
    if (c0 + c < c1) {
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[i] = mfma16(av[c][i], wv[c], acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();
  // wavefront w < MT finishes m-tile w: partials summed in wavefront order
  for (int i = wave; i < MT; i += kLinWaves) {
    f32x4_t t = red[0][i][lane];
#pragma unroll
    for (int w = 1; w < kLinWaves; ++w) t += red[w][i][lane];
    const int n = n0 + j;
    if (n < N) {
      const float bn = bf16_bits_to_f32(bias[n]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + 16 * i + 4 * kb + q;
        if (m < M) {
          const float v = round_bf16(t[q] + bn);
          float o;
          if (EPI == kLinGelu)
            o = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
          else
            o = bf16_bits_to_f32(res[(int64_t)m * N + n]) + v;
          out[(int64_t)m * N + n] = f32_to_bf16_bits(o);
        }
      }
    }
  }
}

hipError_t launch_linear_bf16(int epi, const uint16_t* x, const uint16_t* W, const uint16_t* bias,
                              const uint16_t* res, uint16_t* out, int64_t M, int N, int K,
                              hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (K % 32 != 0 || N <= 0) return hipErrorInvalidValue;
  const int nsteps = K >> 5;
  const int per = (nsteps + kLinWaves - 1) / kLinWaves;
  if (per > kLinMaxSteps) return hipErrorInvalidValue;
  const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  const dim3 grid((N + 15) / 16, (unsigned)((M + 16 * mt - 1) / (16 * mt))), block(64 * kLinWaves);
#define W4A16_LIN(MT_)                                                                            \
  do {                                                                                            \
    if (epi == kLinGelu)                                                                          \
      hipLaunchKernelGGL((k_linear_bf16<MT_, kLinGelu>), grid, block, 0, s, x, W, bias, res, out, \
                         (int)M, N, K, per);                                                      \
    else                                                                                          \
      hipLaunchKernelGGL((k_linear_bf16<MT_, kLinResidual>), grid, block, 0, s, x, W, bias, res,  \
                         out, (int)M, N, K, per);                                                 \
  } while (0)
  if (mt == 1)
    W4A16_LIN(1);
  else if (mt == 2)
    W4A16_LIN(2);
  else
    W4A16_LIN(4);
#undef W4A16_LIN
  return hipGetLastError();
}

}  // namespace w4a16
