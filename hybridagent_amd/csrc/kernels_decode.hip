// Decode-shaped W4A16 kernels for gfx950: few activation rows per weight
// matrix, so the packed weights stream from HBM once and the arithmetic runs
// on 16x16x32 bf16 MFMA tiles.
//
//   k_decode<MODE, BIAS>   one workgroup = 16 weight rows (MFMA columns) of
//                          one expert; its 4 wavefronts split K into 128-wide
//                          tiles (wave w takes tiles w, w+4, ...) and reduce
//                          through LDS.  Each lane streams its weight rows
//                          with 16-byte loads: lanes kb = 0..3 of a column
//                          read 64 contiguous bytes of the row per tile.
//   MODE = dense  : y = x W^T (+bias)                (quantization.py:171-175)
//   MODE = gateup : inter = gelu(x Wg^T) * (x Wu^T)  (quantization.py:112-120)
//                   columns 0..7 of the tile are gate rows n0..n0+7 and
//                   columns 8..15 the matching up rows I+n0..I+n0+7, so the
//                   gated GELU is fused into the epilogue.
//   MODE = down   : dn[t*k+j] = inter W_d^T          (quantization.py:122-127)
//
// k_bias_order, k_combine and k_dequant are the small helpers around it.
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

// ---------------------------------------------------------------------------
// dequantize_int4_packed  (quantization.py:132-137), group size G, ceil groups
// one thread per packed word -> 8 bf16 (16-byte store)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_dequant(const uint32_t* __restrict__ packed,
                                                 const uint16_t* __restrict__ scale,
                                                 uint16_t* __restrict__ out, int64_t rows,
                                                 int K, int G, int ng) {
  const int words = K >> 3;
  const int64_t total = rows * (int64_t)words;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / words;
    const int wj = (int)(i - r * words);
    const float s = bf16_bits_to_f32(scale[r * ng + (wj * 8) / G]);
    st16(out + r * K + wj * 8, unpack_exact<false>(packed[i], s));
  }
}

hipError_t launch_dequant(const int32_t* packed, const uint16_t* scale, uint16_t* out,
                          int64_t rows, int K, int G, hipStream_t s) {
  const int64_t total = rows * (K >> 3);
  if (total == 0) return hipSuccess;
  const int ng = (K + G - 1) / G;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)blocks), dim3(256), 0, s,
                     reinterpret_cast<const uint32_t*>(packed), scale, out, rows, K, G, ng);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// activation rows -> bias order (8-blocks permuted to [0,4,1,5,2,6,3,7])
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_bias_order(const uint16_t* __restrict__ x,
                                                    uint16_t* __restrict__ xp, int64_t n8) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    st16(xp + i * 8, to_bias_order(ld16(x + i * 8)));
  }
}

hipError_t launch_bias_order(const uint16_t* x, uint16_t* xp, int64_t rows, int K,
                             hipStream_t s) {
  const int64_t n8 = rows * (K >> 3);
  if (n8 == 0) return hipSuccess;
  int64_t blocks = (n8 + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_bias_order, dim3((unsigned)blocks), dim3(256), 0, s, x, xp, n8);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// the decode MFMA kernel
// ---------------------------------------------------------------------------
// Operand layout of v_mfma_f32_16x16x32_bf16 as used here: lane l supplies
// A[row l%16][8*(l/16) .. +7] and B[8*(l/16) .. +7][col l%16]; the result lane
// l holds D[4*(l/16) + r][l%16], r = 0..3.  A and B only need to agree on the
// k index carried by (l/16, element), so each lane simply feeds 8 consecutive
// (bias- or natural-ordered) k values of its own 32-element chunk per step.
template <int MODE, bool BIAS>
__global__ __launch_bounds__(256) void k_decode(DecodeArgs a) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int j = lane & 15;   // MFMA column (weight row within the tile) / A row
  const int kb = lane >> 4;  // which 32-element chunk of the 128-wide k tile

  int e = 0, seg0 = 0, rows = a.M;
  if (MODE != kModeDense) {
    const int slot = blockIdx.y;
    if (slot >= *a.n_active) return;  // uniform across the workgroup
    e = a.active[slot];
    seg0 = a.offsets[e];
    rows = a.offsets[e + 1] - seg0;
  }

  int wrow;
  if (MODE == kModeGateUp) {
    const int n0 = blockIdx.x * 8;
    wrow = (j < 8) ? (n0 + j) : (a.I + n0 + (j - 8));
  } else {
    wrow = blockIdx.x * 16 + j;
  }
  const bool col_ok = wrow < a.N;
  const int64_t grow = (int64_t)e * a.N + (col_ok ? wrow : 0);
  const uint32_t* __restrict__ wr = reinterpret_cast<const uint32_t*>(a.wp) + grow * (a.K >> 3);
  const uint16_t* __restrict__ sr = a.ws + grow * a.ng;
  const int nchunks = a.K >> 5;
  const int ntiles = (nchunks + 3) >> 2;

  __shared__ f32x4_t red[4][4][64];

  const u32x4_t c136 = {kBias136Pair, kBias136Pair, kBias136Pair, kBias136Pair};
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};

  for (int mc = 0; mc < rows; mc += 64) {
    const int nmt = min(4, (rows - mc + 15) >> 4);
    const uint16_t* arow[4];
    bool aok[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int i = mc + 16 * mt + j;
      aok[mt] = (mt < nmt) && (i < rows);
      int64_t r = 0;
      if (aok[mt]) {
        if (MODE == kModeDense) r = i;
        else if (MODE == kModeGateUp) r = a.sorted_pos[seg0 + i] / a.topk;
        else r = seg0 + i;
      }
      arow[mt] = a.act + r * a.K;
    }

    f32x4_t acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int t = wave; t < ntiles; t += 4) {
      const int c = 4 * t + kb;
      const bool cok = c < nchunks;
      const u32x4_t bw = (cok && col_ok) ? ld16(wr + 4 * c) : zero4;
      u32x4_t av[4][4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          av[mt][s] = (aok[mt] && cok) ? ld16(arow[mt] + 32 * c + 8 * s) : zero4;
      }
      if (BIAS) {
        // one scale per lane column for the whole 128-wide tile (G % 128 == 0)
        const float sc = col_ok ? bf16_bits_to_f32(sr[(t * 128) / a.G]) : 0.f;
        u32x4_t bv[4];
        bv[0] = unpack_bias(bw.x);
        bv[1] = unpack_bias(bw.y);
        bv[2] = unpack_bias(bw.z);
        bv[3] = unpack_bias(bw.w);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          if (mt < nmt) {
            f32x4_t g = {0.f, 0.f, 0.f, 0.f};
            f32x4_t cr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) g = mfma16(av[mt][s], bv[s], g);
#pragma unroll
            for (int s = 0; s < 4; ++s) cr = mfma16(av[mt][s], c136, cr);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][r] = __builtin_fmaf(sc, g[r] - cr[r], acc[mt][r]);
          }
        }
      } else {
        // each lane's 32-element chunk lies inside one group (G >= 32)
        const float sc = (col_ok && cok) ? bf16_bits_to_f32(sr[(32 * c) / a.G]) : 0.f;
        u32x4_t bv[4];
        bv[0] = unpack_exact<false>(bw.x, sc);
        bv[1] = unpack_exact<false>(bw.y, sc);
        bv[2] = unpack_exact<false>(bw.z, sc);
        bv[3] = unpack_exact<false>(bw.w, sc);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          if (mt < nmt) {
#pragma unroll
            for (int s = 0; s < 4; ++s) acc[mt] = mfma16(av[mt][s], bv[s], acc[mt]);
          }
        }
      }
    }

    // split-K reduction over the 4 wavefronts
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      if (mt < nmt) red[wave][mt][lane] = acc[mt];
    __syncthreads();
    const int mt = wave;  // wavefront w finishes m-tile w
    if (mt < nmt) {
      f32x4_t v = red[0][mt][lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const f32x4_t o = red[w][mt][lane];
        v[0] += o[0]; v[1] += o[1]; v[2] += o[2]; v[3] += o[3];
      }
      const int ibase = mc + 16 * mt + 4 * (lane >> 4);
      if (MODE == kModeDense) {
        const int n = blockIdx.x * 16 + j;
        const float b = (a.bias != nullptr && col_ok) ? bf16_bits_to_f32(a.bias[n]) : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = ibase + r;
          if (col_ok && i < rows) a.out[(int64_t)i * a.N + n] = f32_to_bf16_bits(v[r] + b);
        }
      } else if (MODE == kModeGateUp) {
        // lane j (< 8) holds gate column n0+j, lane j+8 the matching up column
        const int n0 = blockIdx.x * 8;
        const int pos = BIAS ? ((j & 3) * 2 + ((j >> 2) & 1)) : j;  // bias-order slot
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float up = __shfl_xor(v[r], 8);
          const int i = ibase + r;
          if (j < 8 && i < rows) {
            const float gate = round_bf16(v[r]);
            const float act = round_bf16(gelu_tanh_f32(gate));
            const float h = act * round_bf16(up);
            a.out[(int64_t)(seg0 + i) * a.I + n0 + pos] = f32_to_bf16_bits(h);
          }
        }
      } else {
        const int n = blockIdx.x * 16 + j;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = ibase + r;
          if (col_ok && i < rows) {
            const int64_t orow = a.sorted_pos[seg0 + i];
            a.out[orow * a.N + n] = f32_to_bf16_bits(v[r]);
          }
        }
      }
    }
    __syncthreads();
  }
}

hipError_t launch_decode(int mode, bool bias_form, const DecodeArgs& a, int grid_x, int grid_y,
                         hipStream_t s) {
  if (grid_x <= 0 || grid_y <= 0) return hipSuccess;
  dim3 grid(grid_x, grid_y), block(256);
#define W4A16_LAUNCH(M_, B_) hipLaunchKernelGGL((k_decode<M_, B_>), grid, block, 0, s, a)
  if (mode == kModeDense) {
    if (bias_form) W4A16_LAUNCH(kModeDense, true); else W4A16_LAUNCH(kModeDense, false);
  } else if (mode == kModeGateUp) {
    if (bias_form) W4A16_LAUNCH(kModeGateUp, true); else W4A16_LAUNCH(kModeGateUp, false);
  } else {
    if (bias_form) W4A16_LAUNCH(kModeDown, true); else W4A16_LAUNCH(kModeDown, false);
  }
#undef W4A16_LAUNCH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// weighted top-k combine  (quantization.py:128-129)
// y[t] = bf16( sum_j bf16( bf16(w[t,j]) * dn[t*k+j] ) ), fp32 sum in j order.
// Slots whose expert index is outside [0, E) contribute nothing.
// one thread per (token, 8 columns)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_combine(const uint16_t* __restrict__ dn,
                                                 const int64_t* __restrict__ idx,
                                                 const float* __restrict__ w,
                                                 uint16_t* __restrict__ out, int M, int topk,
                                                 int E, int H) {
  const int per_row = H >> 3;
  const int64_t total = (int64_t)M * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / per_row);
    const int c8 = (int)(i - (int64_t)t * per_row) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int jj = 0; jj < topk; ++jj) {
      const int64_t ex = idx[(int64_t)t * topk + jj];
      if (ex < 0 || ex >= E) continue;
      const float wb = round_bf16(w[(int64_t)t * topk + jj]);
      const u32x4_t d = ld16(dn + ((int64_t)t * topk + jj) * H + c8);
      const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += round_bf16(bf16_bits_to_f32(dw[q] & 0xFFFFu) * wb);
        acc[2 * q + 1] += round_bf16(bf16_bits_to_f32(dw[q] >> 16) * wb);
      }
    }
    u32x4_t o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    st16(out + (int64_t)t * H + c8, o);
  }
}

hipError_t launch_combine(const uint16_t* dn, const int64_t* idx, const float* w, uint16_t* out,
                          int M, int topk, int E, int H, hipStream_t s) {
  const int64_t total = (int64_t)M * (H >> 3);
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_combine, dim3((unsigned)blocks), dim3(256), 0, s, dn, idx, w, out, M, topk,
                     E, H);
  return hipGetLastError();
}

}  // namespace w4a16
