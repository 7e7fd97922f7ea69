// bf16-weight linear for small batches (the HybridLink map's projections,
// hybridlink.py:21-22, and the shared MLP of the FFN block,
// backends.py:105-108):
//
//   out[m, n] = epilogue(sum_k x[m, k] W[n, k])     bf16 x [M, K], W [N, K]
//
// The weights stream once: a workgroup owns one 16-column MFMA tile (gate/up:
// 8 gate columns and the same 8 up columns) for up to 64 rows; its eight
// wavefronts split K, each issuing all the weight and activation loads of a
// chunk of up to 12 k steps before the chunk's first MFMA (so a wavefront
// waits for memory once per chunk); the eight partial tiles are summed in
// LDS in wavefront order (deterministic) and the epilogue applies:
//   kLinGelu      bf16(GELU_erf(bf16(acc + b)))                 HybridLink proj1
//   kLinResidual  bf16(res + bf16(acc + b))                     HybridLink proj2
//   kLinGateUp    bf16(bf16(gelu_tanh(bf16(acc_gate))) * bf16(acc_up))
//                 gate rows from W, up rows from W2              shared MLP gate/up
//   kLinPlain     bf16(acc)                                      shared MLP down
// Every rounding point is one of the torch bf16 module's (F.linear rounds its
// output, the activation and the product round theirs).
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kLinWaves = 8;
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

}  // namespace

template <int MT, int EPI>
__global__ __launch_bounds__(64 * kLinWaves) void k_linear_bf16(LinArgs a) {
  __shared__ f32x4_t red[kLinWaves][MT][64];
  constexpr bool GU = EPI == kLinGateUp;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, kb = lane >> 4;
  // gate/up: lanes j < 8 take gate row n0 + j, lanes j >= 8 the up row n0 + j - 8
  const int n0 = blockIdx.x * (GU ? 8 : 16);
  const int m0 = blockIdx.y * 16 * MT;
  const int K = a.K;
  const int nsteps = K >> 5;
  const int c0 = wave * a.steps_per_wave;
  const int c1 = min(nsteps, c0 + a.steps_per_wave);
  // this lane's weight row and activation rows (clamped: columns past N and
  // rows past M compute values that are not stored)
  const uint16_t* wbase = GU && j >= 8 ? a.W2 : a.W;
  const int wr = GU ? n0 + (j & 7) : n0 + j;
  const uint16_t* wrow = wbase + (int64_t)min(wr, a.N - 1) * K + 8 * kb;
  const uint16_t* xrow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) xrow[i] = a.x + (int64_t)min(m0 + 16 * i + j, a.M - 1) * K + 8 * kb;
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
      for (int i = 0; i < MT; ++i) av[c][i] = ld16(xrow[i] + 32 * step_at(c));
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
            a.out[(int64_t)m * a.N + n] = f32_to_bf16_bits(o);
          }
        }
      }
    }
  }
}

hipError_t launch_linear_bf16(int epi, const uint16_t* x, const uint16_t* W, const uint16_t* W2,
                              const uint16_t* bias, const uint16_t* res, uint16_t* out, int64_t M, int N,
                              int K, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (K % 32 != 0 || K <= 0 || N <= 0) return hipErrorInvalidValue;
  const int nsteps = K >> 5;
  LinArgs a{x, W, W2, bias, res, out, (int)M, N, K, (nsteps + kLinWaves - 1) / kLinWaves};
  const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  const int cols = epi == kLinGateUp ? 8 : 16;
  const int64_t gy = (M + 16 * mt - 1) / (16 * mt);
  if (gy > 65535) return hipErrorInvalidValue;
  const dim3 grid((N + cols - 1) / cols, (unsigned)gy), block(64 * kLinWaves);
#define W4A16_LIN(MT_)                                                                     \
  do {                                                                                     \
    switch (epi) {                                                                         \
      case kLinGelu: hipLaunchKernelGGL((k_linear_bf16<MT_, kLinGelu>), grid, block, 0, s, a); break; \
      case kLinResidual: hipLaunchKernelGGL((k_linear_bf16<MT_, kLinResidual>), grid, block, 0, s, a); break; \
      case kLinGateUp: hipLaunchKernelGGL((k_linear_bf16<MT_, kLinGateUp>), grid, block, 0, s, a); break; \
      default: hipLaunchKernelGGL((k_linear_bf16<MT_, kLinPlain>), grid, block, 0, s, a); break; \
    }                                                                                      \
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
