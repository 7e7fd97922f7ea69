// Body of the bf16-weight linear for small batches (k_linear_bf16 in
// kernels_linear_bf16.hip; the FFN block's router launches also run it in
// their spare workgroups).  One workgroup of kLinWaves wavefronts computes
// the output block (bx, by): one 16-column MFMA tile (gate/up: 8 gate
// columns and the same 8 up columns) for up to 16 * MT rows.
//
// Fragment order (the HybridLink chain's activations, kLinGelu's input and
// output, kLinResidual's input): rows padded to a multiple of 16, element
// (m, k) of a [Mp, K] matrix at
//   ((m / 16) * (K / 32) + k / 32) * 512 + ((k % 32) / 8) * 128 + (m % 16) * 8 + k % 8,
// so the 16 rows x 32 k of one MFMA step's A operand are one contiguous KiB
// (lane l's 16 bytes at 16 l) instead of 16 rows x 64 bytes: the activation
// loads read whole cache lines (measured: a 2816 x 2816 linear at M = 32
// 11.4 -> 7.9 us).  Rows past M in the padding hold whatever the buffer
// held; they reach only output rows that are not stored.
#pragma once
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

constexpr int kLinWaves = 8;
constexpr int kLinThreads = 64 * kLinWaves;
constexpr int kLinMaxSteps = 12;  // 32-wide k steps per wavefront held in registers

struct LinArgs {
  const uint16_t* x;
  const uint16_t* W;
  const uint16_t* W2;    // kLinGateUp: the up rows
  const uint16_t* bias;  // kLinGelu / kLinResidual
  const uint16_t* res;   // kLinResidual
  uint16_t* out;
  int M, N, K, steps_per_wave;
};

// row tiles of 16 per workgroup for M rows, and the grid of the launch
inline int lin_row_tiles(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }
inline LinArgs lin_args(int, const uint16_t* x, const uint16_t* W, const uint16_t* W2, const uint16_t* bias,
                        const uint16_t* res, uint16_t* out, int64_t M, int N, int K) {
  const int nsteps = K >> 5;
  return LinArgs{x, W, W2, bias, res, out, (int)M, N, K, (nsteps + kLinWaves - 1) / kLinWaves};
}
inline int lin_grid_x(int epi, int N) { return (N + (epi == kLinGateUp ? 8 : 16) - 1) / (epi == kLinGateUp ? 8 : 16); }
inline int64_t lin_grid_y(int64_t M) { return (M + 16 * lin_row_tiles(M) - 1) / (16 * lin_row_tiles(M)); }

// element (m, k) of a fragment-order matrix with K columns
__host__ __device__ inline int64_t frag_index(int64_t m, int k, int K) {
  return ((m >> 4) * (K >> 5) + (k >> 5)) * 512 + ((k & 31) >> 3) * 128 + (m & 15) * 8 + (k & 7);
}
// the epilogues whose input (XF) and output (OF) are in fragment order
constexpr bool lin_x_frag(int epi) { return epi == kLinGelu || epi == kLinResidual; }
constexpr bool lin_out_frag(int epi) { return epi == kLinGelu; }

template <int MT, int EPI>
__device__ __forceinline__ void linear_bf16_block(const LinArgs& a, int bx, int by) {
  __shared__ f32x4_t red[kLinWaves][MT][64];
  constexpr bool GU = EPI == kLinGateUp;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, kb = lane >> 4;
  // gate/up: lanes j < 8 take gate row n0 + j, lanes j >= 8 the up row n0 + j - 8
  const int n0 = bx * (GU ? 8 : 16);
  const int m0 = by * 16 * MT;
  const int K = a.K;
  const int nsteps = K >> 5;
  const int c0 = wave * a.steps_per_wave;
  const int c1 = min(nsteps, c0 + a.steps_per_wave);
  // this lane's weight row and activation rows (clamped: columns past N and
  // rows past M compute values that are not stored)
  const uint16_t* wbase = GU && j >= 8 ? a.W2 : a.W;
  const int wr = GU ? n0 + (j & 7) : n0 + j;
  const uint16_t* wrow = wbase + (int64_t)min(wr, a.N - 1) * K + 8 * kb;
  // fragment order: the m-tile's piece of step c at 512 c + 8 lane (the
  // padding holds every m-tile a launch touches)
  constexpr bool XF = lin_x_frag(EPI);
  constexpr int XSTEP = XF ? 512 : 32;
  const uint16_t* xrow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
    xrow[i] = XF ? a.x + (int64_t)(min(m0 + 16 * i, a.M - 1) >> 4) * nsteps * 512 + 8 * lane
                 : a.x + (int64_t)min(m0 + 16 * i + j, a.M - 1) * K + 8 * kb;
  f32x4_t acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // chunks of up to kLinMaxSteps k steps: every load of the chunk before its
  // first MFMA -- the weights (HBM), then the activation fragments
  // (L2-resident).  Steps past the range load its last step again (unused).
  for (int cb = c0; cb < c1; cb += kLinMaxSteps) {
    const int ce = min(c1, cb + kLinMaxSteps);
    auto step_at = [&](int c) { return min(cb + c, ce - 1); };
    u32x4_t wv[kLinMaxSteps];
#pragma unroll
    for (int c = 0; c < kLinMaxSteps; ++c) wv[c] = ld16(wrow + 32 * step_at(c));
    u32x4_t av[kLinMaxSteps][MT];
#pragma unroll
    for (int c = 0; c < kLinMaxSteps; ++c)
#pragma unroll
      for (int i = 0; i < MT; ++i) av[c][i] = ld16(xrow[i] + XSTEP * step_at(c));
#pragma unroll
    for (int c = 0; c < kLinMaxSteps; ++c) {
      if (cb + c < ce) {
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i] = mfma16(av[c][i], wv[c], acc[i]);
      }
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
    if (GU) {
      // lane j < 8 holds gate column n0 + j, lane j + 8 the matching up column
      float up[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) up[q] = lane_xor8(t[q]);
      const int n = n0 + j;
      if (j < 8 && n < a.N) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = m0 + 16 * i + 4 * kb + q;
          if (m < a.M) {
            const float gate = round_bf16(t[q]);
            const float act = round_bf16(gelu_tanh_f32(gate));
            a.out[(int64_t)m * a.N + n] = f32_to_bf16_bits(act * round_bf16(up[q]));
          }
        }
      }
    } else {
      const int n = n0 + j;
      if (n < a.N) {
        const float bn = (EPI == kLinGelu || EPI == kLinResidual) ? bf16_bits_to_f32(a.bias[n]) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = m0 + 16 * i + 4 * kb + q;
          if (m < a.M) {
            float o;
            if (EPI == kLinPlain) {
              o = t[q];
            } else {
              const float v = round_bf16(t[q] + bn);
              if (EPI == kLinGelu)
                o = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
              else
                o = bf16_bits_to_f32(a.res[(int64_t)m * a.N + n]) + v;
            }
            a.out[lin_out_frag(EPI) ? frag_index(m, n, a.N) : (int64_t)m * a.N + n] = f32_to_bf16_bits(o);
          }
        }
      }
    }
  }
}


}  // namespace w4a16
