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
#include "linear_bf16.hpp"

namespace w4a16 {

template <int MT, int EPI>
__global__ __launch_bounds__(kLinThreads) void k_linear_bf16(LinArgs a) {
  linear_bf16_block<MT, EPI>(a, blockIdx.x, blockIdx.y);
}

hipError_t launch_linear_bf16(int epi, const uint16_t* x, const uint16_t* W, const uint16_t* W2,
                              const uint16_t* bias, const uint16_t* res, uint16_t* out, int64_t M, int N,
                              int K, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (K % 32 != 0 || K <= 0 || N <= 0) return hipErrorInvalidValue;
  const LinArgs a = lin_args(epi, x, W, W2, bias, res, out, M, N, K);
  const int mt = lin_row_tiles(M);
  const int64_t gy = lin_grid_y(M);
  if (gy > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)lin_grid_x(epi, N), (unsigned)gy), block(kLinThreads);
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
