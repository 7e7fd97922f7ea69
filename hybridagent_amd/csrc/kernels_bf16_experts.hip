// Grouped GEMMs of the BF16 experts path (_bf16_experts_fast_forward,
// backends.py:209-283): the unquantised Gemma4TextExperts weights
// gate_up_proj [E, 2I, H] and down_proj [E, H, I] (bf16), on the expert
// segments the MoE plan (k_moe_sort) produced:
//
//   MODE = gateup : inter[s] = bf16(bf16(gelu_tanh(bf16(x[tok(s)] Wg^T))) * bf16(x[tok(s)] Wu^T))
//                   (backends.py:224-232, 243-252, 274-276), rows s in segment order
//   MODE = down   : dn[sorted_pos[s]] = bf16(inter[s] W_d^T)   (:234-237, 254-259, 277)
//
// then k_combine forms the weighted top-k sum.  Grid (group of CB column
// blocks, active expert slot); a workgroup whose slot is past the active
// count leaves at once.  Its eight wavefronts are CB column blocks x KS = 8 /
// CB ranges of K: each streams its block's weights over its K range (16-byte
// loads, every load of a 12-step chunk of k issued before its first MFMA)
// once per chunk of 16, 32 or 64 rows of the expert's segment (sized from
// the mean rows per expert); the KS partial tiles of a block are summed in
// LDS in K order and the epilogue writes bf16 rows.  gate_up blocks pair 8
// gate columns with the same 8 up columns, so the gated GELU is formed in
// registers.  Several blocks per workgroup amortise its fixed costs (the
// row positions, the reduction, the epilogue) over more weight bytes: down
// (K = 704) takes 4 blocks of 2 K ranges, gate_up 2 blocks of 4.
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kBfWaves = 8;
constexpr int kBfMaxSteps = 12;  // 32-wide k steps per wavefront per chunk

}  // namespace

// MT: 16-row m-tiles per row chunk, chosen from the expected rows per expert
// (the activation fragments of a chunk live in registers: 48 MT VGPRs);
// CB: column blocks per workgroup (KS = 8 / CB wavefronts per block split K)
template <int MODE, int MT, int CB>
__global__ __launch_bounds__(64 * kBfWaves) void k_bf16_expert(Bf16ExpertArgs a) {
  constexpr int KS = kBfWaves / CB;
  __shared__ f32x4_t red[kBfWaves][MT][64];
  __shared__ int rowsrc[16 * MT];
  const int slot = blockIdx.y;
  if (slot >= ld_uniform(a.n_active, 0)) return;
  const int e = ld_uniform(a.desc, 4 * slot);
  const int seg0 = ld_uniform(a.desc, 4 * slot + 1);
  const int rows = ld_uniform(a.desc, 4 * slot + 2);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cb = wave / KS, ks = wave - cb * KS;
  const int j = lane & 15, kb = lane >> 4;
  constexpr bool GU = MODE == kModeGateUp;
  const int ncols = GU ? a.I : a.N;  // output columns
  // this wavefront's block: gate_up lanes j < 8 take gate row n0 + j, lanes
  // j >= 8 up row I + n0 + j - 8; blocks past the matrix read its last row
  // and store nothing
  const int n0 = (blockIdx.x * CB + cb) * (GU ? 8 : 16);
  const int K = a.K;
  const int nsteps = K >> 5;
  const int per = (nsteps + KS - 1) / KS;
  const int c0 = ks * per;
  const int c1 = min(nsteps, c0 + per);
  const int wr = GU ? (j < 8 ? n0 + j : a.I + n0 + (j - 8)) : n0 + j;
  const uint16_t* wrow = a.W + ((int64_t)e * a.N + min(wr, a.N - 1)) * K + 8 * kb;
  for (int r0 = 0; r0 < rows; r0 += 16 * MT) {
    const int nr = min(16 * MT, rows - r0);
    __syncthreads();  // the previous chunk's readers of rowsrc / red are done
    if (threadIdx.x < 16 * MT) {
      const int i = min((int)threadIdx.x, nr - 1);
      const int sp = a.sorted_pos[seg0 + r0 + i];
      rowsrc[threadIdx.x] = GU ? sp / a.topk : seg0 + r0 + i;
    }
    __syncthreads();
    const uint16_t* xrow[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) xrow[i] = a.act + (int64_t)rowsrc[16 * i + j] * K + 8 * kb;
    f32x4_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int cc = c0; cc < c1; cc += kBfMaxSteps) {
      const int ce = min(c1, cc + kBfMaxSteps);
      auto step_at = [&](int c) { return min(cc + c, ce - 1); };
      u32x4_t wv[kBfMaxSteps];
#pragma unroll
      for (int c = 0; c < kBfMaxSteps; ++c) wv[c] = ld16(wrow + 32 * step_at(c));
      u32x4_t av[kBfMaxSteps][MT];
#pragma unroll
      for (int c = 0; c < kBfMaxSteps; ++c)
#pragma unroll
        for (int i = 0; i < MT; ++i) av[c][i] = ld16(xrow[i] + 32 * step_at(c));
#pragma unroll
      for (int c = 0; c < kBfMaxSteps; ++c) {
        if (cc + c < ce) {
#pragma unroll
          for (int i = 0; i < MT; ++i) acc[i] = mfma16(av[c][i], wv[c], acc[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    // wavefront (cb, ks) finishes m-tiles i = ks, ks + KS, ... of its block:
    // the block's partials summed in K order
    for (int i = ks; i < MT; i += KS) {
      f32x4_t t = red[cb * KS][i][lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) t += red[cb * KS + w][i][lane];
      if (GU) {
        float up[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) up[q] = lane_xor8(t[q]);
        const int n = n0 + j;
        if (j < 8 && n < ncols) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = 16 * i + 4 * kb + q;
            if (r < nr) {
              const float gate = round_bf16(t[q]);
              const float act = round_bf16(gelu_tanh_f32(gate));
              a.out[(int64_t)(seg0 + r0 + r) * a.I + n] = f32_to_bf16_bits(act * round_bf16(up[q]));
            }
          }
        }
      } else {
        const int n = n0 + j;
        if (n < ncols) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = 16 * i + 4 * kb + q;
            if (r < nr) a.out[(int64_t)a.sorted_pos[seg0 + r0 + r] * a.N + n] = f32_to_bf16_bits(t[q]);
          }
        }
      }
    }
  }
}

hipError_t launch_bf16_experts(int mode, Bf16ExpertArgs a, int max_slots, hipStream_t s) {
  if (max_slots <= 0) return hipSuccess;
  if (a.K % 32 != 0 || a.K <= 0 || max_slots > 65535) return hipErrorInvalidValue;
  // column blocks per workgroup: down 4 (K splits of 2), gate_up 2 (of 4)
  const int cbk = mode == kModeGateUp ? 2 : 4;
  const int cols = (mode == kModeGateUp ? 8 : 16) * cbk;
  const int ncols = mode == kModeGateUp ? a.I : a.N;
  const dim3 grid((ncols + cols - 1) / cols, (unsigned)max_slots), block(64 * kBfWaves);
  // rows per expert on average: M * topk / E (the sort's segments)
  const int64_t avg = (int64_t)a.rows_total / (max_slots > 0 ? max_slots : 1);
#define W4A16_BF(MT_)                                                                   \
  do {                                                                                  \
    if (mode == kModeGateUp)                                                            \
      hipLaunchKernelGGL((k_bf16_expert<kModeGateUp, MT_, 2>), grid, block, 0, s, a);   \
    else                                                                                \
      hipLaunchKernelGGL((k_bf16_expert<kModeDown, MT_, 4>), grid, block, 0, s, a);     \
  } while (0)
  if (avg <= 16)
    W4A16_BF(1);
  else if (avg <= 32)
    W4A16_BF(2);
  else
    W4A16_BF(4);
#undef W4A16_BF
  return hipGetLastError();
}

}  // namespace w4a16
