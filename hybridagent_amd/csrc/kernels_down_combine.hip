// Decode sizes (at most 64 routed rows): the down projection and the
// weighted top-k combine in one launch (quantization.py:122-129),
//
//   y[t, n] = bf16( sum_j bf16( bf16(w[t, j]) * dn[t*k + j, n] ) ),
//   dn[t*k + j, n] = bf16( inter[s] . W_e[n] ),  s the segment row of (t, j),
//
// with the products summed in j order as the separate combine does, so the
// result equals the down streamer followed by k_combine bit for bit (the
// same MFMA operand layout, the same per-tile fold order).
//
// The separate path needs every expert's down output in memory before the
// combine launch can read it; here one workgroup owns 16 output columns of
// every token, so it sees all k slots of a token and combines them in LDS.
// Workgroup b: columns 16 b .. 16 b + 15 of every active expert.  It stages
// all routed intermediate rows in LDS (fragment order, as the streamer does),
// then its eight wavefronts take the active experts in turn (wavefront w:
// slots w, w + 8, ...): per expert 16-row MFMA tiles over the whole K,
// the next expert's weight loads in flight during the current one's MFMAs.
// Each result row goes into LDS as its weighted product, at the row's place
// t * k + j; after a barrier each thread sums one (token, column).
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kDcWaves = 8;
constexpr int kDcThreads = 64 * kDcWaves;
constexpr int kDcCols = 16;
constexpr int kDcTiles = 6;  // k tiles of 128 per row (K <= 768)

// 16-byte piece b (elements 8 b .. 8 b + 7) of staged row r: grouped by
// (k tile, lane chunk, MFMA step) like the streamer, rows innermost
__device__ __forceinline__ int dc_slot(int b, int R, int r) {
  return (16 * (b >> 4) + 4 * (b & 3) + ((b >> 2) & 3)) * R + r;
}

}  // namespace

// The intermediate rows are in bias order (what the decode gate_up epilogue
// writes).  FORM says how the weights are read and unpacked:
//   kDcExact  packed layout, exact dequantisation bf16_RNE((u - 8) * s) in
//             bias order (group sizes below 128);
//   kDcBias   packed layout, bf16(128 + u), the fold subtracts 136 * the
//             tile's row sum and applies the group scale (group size a
//             multiple of 128);
//   kDcTiled  as kDcBias on the down streamer's tiled copy (group size 128);
//   kDcStep   the tiled copy of group size 32 / 64 (bias-form build): each
//             MFMA step one 32-wide chunk, folded with its own scale (from
//             the copy);
//   kDcExactTiled  as kDcExact on the down streamer's tiled copy (group size
//             128: scales from the scale tensor; 32 / 64: from the copy).
enum { kDcExact = 0, kDcBias = 1, kDcTiled = 2, kDcStep = 3, kDcExactTiled = 4 };

template <int FORM>
__global__ __launch_bounds__(kDcThreads) void k_down_combine(DownCombineArgs a) {
  constexpr bool BIAS = FORM == kDcBias || FORM == kDcTiled || FORM == kDcStep;
  constexpr bool TILED = FORM == kDcTiled || FORM == kDcStep || FORM == kDcExactTiled;
  constexpr bool STEP = FORM == kDcStep;
  constexpr int NCS = STEP ? 4 : 1;  // corrections per k tile
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int R = a.M * a.topk;  // routed rows (<= kDownCombineMaxRows)
  const int K8 = a.K >> 3;
  const int ntiles = (K8 + 15) >> 4;
  u32x4_t* __restrict__ xs = reinterpret_cast<u32x4_t*>(smem_raw);             // [16 ntiles][R]
  float* __restrict__ csum = reinterpret_cast<float*>(smem_raw + (size_t)16 * kDcTiles * R * 16);  // [NCS ntiles][R]
  float* __restrict__ prod = csum + NCS * kDcTiles * R;                          // [R][16]
  int* __restrict__ slot_pos = reinterpret_cast<int*>(prod + R * kDcCols);       // [threads]: t*k+j of segment row s
  float* __restrict__ wts = reinterpret_cast<float*>(slot_pos + kDcThreads);      // [threads]: bf16(w[t, j]) at t*k+j
  int* __restrict__ has_e = reinterpret_cast<int*>(wts + kDcThreads);            // [threads]: slot t*k+j has an expert
  // LDS slot of 16-byte piece b of staged row r: STEP keeps pieces in order
  // (step s of tile t reads pieces 16 t + 4 s + kb), the others group them by
  // (k tile, lane chunk, MFMA step) like the streamer
  auto slot = [&](int b, int r) { return STEP ? b * R + r : dc_slot(b, R, r); };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15;   // MFMA column: weight row n0 + j; A row
  const int kb = lane >> 4;  // 32-element chunk of a 128-wide k tile
  const int n0 = (int)blockIdx.x * kDcCols;
  const int U = ld_uniform(a.n_active, 0);

  // one expert's 16 weight rows (this lane: row n0 + j) over all of K and
  // their scales.  Packed: the 32-element chunk kb of every k tile, one
  // scale per tile (bias) or chunk (exact).  Tiled: this workgroup's 16
  // rows are the copy's block blockIdx.x (16-row column block of the down
  // streamer, no K split), tile t at KiB t, lane l's 16 bytes at 16 l; tiles
  // past the copy's TPW read the block's first KiB with a zero scale.
  // STEP: sc holds the block's step scales of row j, two tiles per entry.
  const int wrow = min(n0 + j, a.N - 1);
  const uint32_t mat_bytes = TILED ? (uint32_t)a.expert_bytes : (uint32_t)a.N * (uint32_t)K8 * 4u;
  const int blk = (int)blockIdx.x * a.block_bytes;
  using ScT = typename std::conditional<STEP, u32x4_t, uint32_t>::type;
  auto weights = [&](int u, u32x4_t* bw, ScT* sc) {
    const int e = min(max(ld_uniform(a.desc, 4 * u), 0), a.E - 1);
    const __amdgpu_buffer_rsrc_t wsrc =
        TILED ? make_rsrc(reinterpret_cast<const unsigned char*>(a.wt) + (int64_t)e * a.expert_bytes, mat_bytes)
              : make_rsrc(reinterpret_cast<const uint32_t*>(a.wp) + (int64_t)e * a.N * K8, mat_bytes);
    const __amdgpu_buffer_rsrc_t ssrc = make_rsrc(a.ws + (int64_t)e * a.N * a.ng, (uint32_t)a.N * a.ng * 2u);
#pragma unroll
    for (int t = 0; t < kDcTiles; ++t) {
      if (TILED) {
        bw[t] = buf_ld16(wsrc, blk + 16 * lane, t < a.tpw ? 1024 * t : 0);
      } else {
        bw[t] = buf_ld16(wsrc, wrow * K8 * 4 + 64 * t + 16 * kb, 0);
      }
      if constexpr (STEP) {
        if (t & 1) sc[t >> 1] = buf_ld16(wsrc, blk + a.tpw * 1024 + j * (a.tpw * 8), 16 * min(t >> 1, a.tpw / 2 - 1));
      } else if (FORM == kDcExactTiled && a.G != 128) {
        // the copy's lane scales: this lane's chunk in each tile
        sc[t] = (uint32_t)buf_ld_u16(wsrc, blk + a.tpw * 1024 + lane * (a.tpw * 2) + 2 * min(t, a.tpw - 1));
      } else {
        const int g = BIAS ? (t * 128) / a.G : ((4 * t + kb) * 32) / a.G;
        sc[t] = (uint32_t)buf_ld_u16(ssrc, (wrow * a.ng + min(g, a.ng - 1)) * 2);
      }
    }
  };
  // Stage every routed row: one thread per (row, k tile) -- at most 64 x 6
  // tasks -- its 16 pieces (pieces past K are zero), summed as the
  // streamer does: the two halves of 8 pieces in piece order, then added
  // (STEP: each 32-wide chunk's 4 pieces).
  // The row loads are issued first, then this wavefront's first expert's
  // weights, so waiting for the rows does not wait for the weights.
  // Every load is issued unconditionally (threads without a task, and
  // wavefronts without such an expert, load valid data they discard), so
  // the compiler's waits count exactly and waiting for the rows does not
  // wait for the weights issued after them.
  const bool has = tid < R * ntiles;
  const int task = has ? tid : 0;
  const int sr = task / ntiles;
  const int st = task - sr * ntiles;
  const int nb = min(16, K8 - 16 * st);
  u32x4_t v[16];
  {
    const uint16_t* src = a.act + (int64_t)sr * a.K + 128 * st;
#pragma unroll
    for (int b = 0; b < 16; ++b) v[b] = ld16(src + 8 * min(b, nb - 1));
  }
  const int spos = a.sorted_pos[min(tid, R - 1)];
  const float wrt = a.topk_w[min(tid, R - 1)];
  const int64_t ex = a.topk_idx[min(tid, R - 1)];
  // (scales kept 32 bits wide: packing two 16-bit loads into one register
  // would wait for both where the loop carries them)
  constexpr int NSC = STEP ? kDcTiles / 2 : kDcTiles;
  u32x4_t bw0[kDcTiles], bw1[kDcTiles];
  ScT sc0[NSC], sc1[NSC];
  __builtin_amdgcn_sched_barrier(0);
  weights(max(min(wave, U - 1), 0), bw0, sc0);
  __builtin_amdgcn_sched_barrier(0);
  slot_pos[tid] = spos;  // entries past R are not read
  wts[tid] = round_bf16(wrt);
  has_e[tid] = ex >= 0 && ex < a.E;
  auto rowsum = [](const u32x4_t& x) {
    return bf16_bits_to_f32(x.x & 0xFFFFu) + bf16_bits_to_f32(x.x >> 16) + bf16_bits_to_f32(x.y & 0xFFFFu) +
           bf16_bits_to_f32(x.y >> 16) + bf16_bits_to_f32(x.z & 0xFFFFu) + bf16_bits_to_f32(x.z >> 16) +
           bf16_bits_to_f32(x.w & 0xFFFFu) + bf16_bits_to_f32(x.w >> 16);
  };
  if (has) {
    float half[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const u32x4_t x = b < nb ? v[b] : u32x4_t{0u, 0u, 0u, 0u};
      if (BIAS) half[STEP ? b >> 2 : b >> 3] += rowsum(x);
      xs[slot(16 * st + b, sr)] = x;
    }
    if (STEP) {
#pragma unroll
      for (int c = 0; c < 4; ++c) csum[(4 * st + c) * R + sr] = 136.0f * half[c];
    } else if (BIAS) {
      csum[st * R + sr] = 136.0f * (half[0] + half[1]);
    }
  }
  __syncthreads();

  const uint32_t kMask = opaque(0x000F000Fu), kBias = opaque(kBiasPair);
  const ExactRegs kr = exact_regs();
  // one expert's rows times its 16 x K weight tile (in bw / sc), in 16-row
  // MFMA tiles -- more than 16 rows only when tokens route several of their
  // k slots to one expert -- the weighted rows into prod
  auto expert = [&](int u, const u32x4_t* bw, const ScT* sc) {
    const int seg = ld_uniform(a.desc, 4 * u + 1);
    const int seg_rows = ld_uniform(a.desc, 4 * u + 2);
    for (int c0 = 0; c0 < seg_rows; c0 += 16) {
    const int seg0 = seg + c0;
    const int rows = min(16, seg_rows - c0);
    const int ar = seg0 + min(j, rows - 1);  // A row of this lane (rows past the tile: discarded)
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kDcTiles; ++t) {
      const bool t_ok = t < ntiles;
      const int tc = t_ok ? t : ntiles - 1;
      u32x4_t A[4];
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) A[s2] = xs[slot(STEP ? 16 * tc + 4 * s2 + kb : 16 * tc + 4 * kb + s2, ar)];
      const u32x4_t w4 = bw[t];
      if constexpr (STEP) {
        const u32x4_t bv[4] = {unpack_bias(w4.x, kMask, kBias), unpack_bias(w4.y, kMask, kBias),
                               unpack_bias(w4.z, kMask, kBias), unpack_bias(w4.w, kMask, kBias)};
        f32x4_t g[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) g[s2] = mfma16(A[s2], bv[s2], f32x4_t{0.f, 0.f, 0.f, 0.f});
        const uint32_t d0 = (t & 1) ? sc[t >> 1].z : sc[t >> 1].x;
        const uint32_t d1 = (t & 1) ? sc[t >> 1].w : sc[t >> 1].y;
        const float ss[4] = {__uint_as_float(d0 << 16), __uint_as_float(d0 & 0xFFFF0000u),
                             __uint_as_float(d1 << 16), __uint_as_float(d1 & 0xFFFF0000u)};
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          const float scs = (t_ok && t < a.tpw) ? ss[s2] : 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float cr = csum[(4 * tc + s2) * R + seg0 + min(4 * kb + q, rows - 1)];
            acc[q] = __builtin_fmaf(scs, g[s2][q] - cr, acc[q]);
          }
        }
      } else if (BIAS) {
        const float sci = (t_ok && (!TILED || t < a.tpw)) ? bf16_bits_to_f32(sc[t]) : 0.f;
        const u32x4_t bv[4] = {unpack_bias(w4.x, kMask, kBias), unpack_bias(w4.y, kMask, kBias),
                               unpack_bias(w4.z, kMask, kBias), unpack_bias(w4.w, kMask, kBias)};
        f32x4_t g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) g = mfma16(A[s2], bv[s2], g);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float cr = csum[tc * R + seg0 + min(4 * kb + q, rows - 1)];
          acc[q] = __builtin_fmaf(sci, g[q] - cr, acc[q]);
        }
      } else {
        const bool s_ok = t_ok && 4 * t + kb < (a.K >> 5) && (!TILED || t < a.tpw);
        const ExactScale es = exact_scale(s_ok ? bf16_bits_to_f32(sc[t]) : 0.f);
        const u32x4_t bv[4] = {unpack_exact<true>(w4.x, es, kr), unpack_exact<true>(w4.y, es, kr),
                               unpack_exact<true>(w4.z, es, kr), unpack_exact<true>(w4.w, es, kr)};
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) acc = mfma16(A[s2], bv[s2], acc);
      }
    }
    // result rows 4 kb + q: bf16 down output times the rounded routing
    // weight, rounded, at the row's place t*k + j
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = 4 * kb + q;
      if (i < rows && n0 + j < a.N) {
        const int pos = slot_pos[seg0 + i];
        prod[pos * kDcCols + j] = round_bf16(round_bf16(acc[q]) * wts[pos]);
      }
    }
    }
  };
  // slots u, u + 8 with the two register sets; each set is refilled with
  // the slot two steps ahead right after it has been used (a third set,
  // two slots in flight, measured slower)
  for (int u = wave; u < U; u += 2 * kDcWaves) {
    weights(min(u + kDcWaves, U - 1), bw1, sc1);
    expert(u, bw0, sc0);
    weights(min(u + 2 * kDcWaves, U - 1), bw0, sc0);
    if (u + kDcWaves < U) expert(u + kDcWaves, bw1, sc1);
  }
  __syncthreads();

  // one thread per (token, column): the slots' products in j order
  for (int o = tid; o < a.M * kDcCols; o += kDcThreads) {
    const int t = o / kDcCols;
    const int c = o - t * kDcCols;
    if (n0 + c >= a.N) continue;
    float y = 0.f;
    for (int jj = 0; jj < a.topk; ++jj) {
      const int r = t * a.topk + jj;
      if (has_e[r]) y += prod[r * kDcCols + c];
    }
    a.out[(int64_t)t * a.N + n0 + c] = f32_to_bf16_bits(y);
  }
}

size_t down_combine_lds(int rows, bool step) {
  return (size_t)16 * kDcTiles * rows * 16 + (size_t)kDcTiles * rows * 4 * (step ? 4 : 1) +
         (size_t)rows * kDcCols * 4 + (size_t)kDcThreads * 12;
}

// all routed rows fit the LDS stage (an expert's rows go through 16-row
// MFMA tiles, so any routing -- one token's slots on one expert too -- fits)
bool down_combine_supported(int64_t M, int64_t topk, int64_t K) {
  return M > 0 && M * topk <= kDownCombineMaxRows && K % 32 == 0 && K <= 128 * kDcTiles;
}

hipError_t launch_down_combine(DownCombineArgs a, hipStream_t s) {
  const int rows = a.M * a.topk;
  if (rows == 0) return hipSuccess;
  if (!down_combine_supported(a.M, a.topk, a.K)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.N + kDcCols - 1) / kDcCols));
  int form = kDecodeBiasForm && a.G % 128 == 0 ? kDcBias : kDcExact;
  if (a.wt != nullptr) {
    // the tiled copy's blocks are the 16-row column blocks, TPW <= 6 tiles
    if (a.tpw <= 0 || a.tpw > kDcTiles || a.tpw % 2 != 0) return hipErrorInvalidValue;
    form = !kDecodeBiasForm ? kDcExactTiled : a.G == 128 ? kDcTiled : kDcStep;
  }
  const size_t lds = down_combine_lds(rows, form == kDcStep);
  switch (form) {
    case kDcExact: hipLaunchKernelGGL(k_down_combine<kDcExact>, grid, dim3(kDcThreads), lds, s, a); break;
    case kDcBias: hipLaunchKernelGGL(k_down_combine<kDcBias>, grid, dim3(kDcThreads), lds, s, a); break;
    case kDcTiled: hipLaunchKernelGGL(k_down_combine<kDcTiled>, grid, dim3(kDcThreads), lds, s, a); break;
    case kDcExactTiled:
      hipLaunchKernelGGL(k_down_combine<kDcExactTiled>, grid, dim3(kDcThreads), lds, s, a);
      break;
    default: hipLaunchKernelGGL(k_down_combine<kDcStep>, grid, dim3(kDcThreads), lds, s, a); break;
  }
  return hipGetLastError();
}

}  // namespace w4a16
