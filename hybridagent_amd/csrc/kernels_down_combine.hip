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

// The intermediate rows are in the order (0,4,1,5,2,6,3,7) per 8 columns
// (what the decode gate_up epilogue writes); the weights are dequantised
// exactly, bf16_RNE((u - 8) * s), and unpacked in that order.  TILED reads
// them from the down streamer's tiled copy (group size 128: scales from the
// scale tensor; 32 / 64: from the copy), otherwise from the packed layout.
template <bool TILED>
__global__ __launch_bounds__(kDcThreads) void k_down_combine(DownCombineArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int R = a.M * a.topk;  // routed rows (<= kDownCombineMaxRows)
  const int K8 = a.K >> 3;
  const int ntiles = (K8 + 15) >> 4;
  u32x4_t* __restrict__ xs = reinterpret_cast<u32x4_t*>(smem_raw);                    // [16 ntiles][R]
  float* __restrict__ prod = reinterpret_cast<float*>(smem_raw + (size_t)16 * kDcTiles * R * 16);  // [R][16]
  int* __restrict__ slot_pos = reinterpret_cast<int*>(prod + R * kDcCols);       // [threads]: t*k+j of segment row s
  float* __restrict__ wts = reinterpret_cast<float*>(slot_pos + kDcThreads);      // [threads]: bf16(w[t, j]) at t*k+j
  int* __restrict__ has_e = reinterpret_cast<int*>(wts + kDcThreads);            // [threads]: slot t*k+j has an expert

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15;   // MFMA column: weight row n0 + j; A row
  const int kb = lane >> 4;  // 32-element chunk of a 128-wide k tile
  const int n0 = (int)blockIdx.x * kDcCols;
  const int U = ld_uniform(a.n_active, 0);

  // one expert's 16 weight rows (this lane: row n0 + j) over all of K and
  // their scales, one per 32-element chunk.  Packed: the chunk kb of every
  // k tile.  Tiled: this workgroup's 16 rows are the copy's block blockIdx.x
  // (16-row column block of the down streamer, no K split), tile t at KiB t,
  // lane l's 16 bytes at 16 l; tiles past the copy's TPW read the block's
  // first KiB with a zero scale.
  const int wrow = min(n0 + j, a.N - 1);
  const uint32_t mat_bytes = TILED ? (uint32_t)a.expert_bytes : (uint32_t)a.N * (uint32_t)K8 * 4u;
  const int blk = (int)blockIdx.x * a.block_bytes;
  auto weights = [&](int u, u32x4_t* bw, uint32_t* sc) {
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
      if (TILED && a.G != 128) {
        // the copy's lane scales: this lane's chunk in each tile
        sc[t] = (uint32_t)buf_ld_u16(wsrc, blk + a.tpw * 1024 + lane * (a.tpw * 2) + 2 * min(t, a.tpw - 1));
      } else {
        const int g = ((4 * t + kb) * 32) / a.G;
        sc[t] = (uint32_t)buf_ld_u16(ssrc, (wrow * a.ng + min(g, a.ng - 1)) * 2);
      }
    }
  };
  // Stage every routed row: one thread per (row, k tile) -- at most 64 x 6
  // tasks -- its 16 pieces (pieces past K are zero).
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
  u32x4_t bw0[kDcTiles], bw1[kDcTiles];
  uint32_t sc0[kDcTiles], sc1[kDcTiles];
  __builtin_amdgcn_sched_barrier(0);
  // the first slot's descriptor is read without waiting for the active
  // count: a wavefront past the active slots loads (clamped, in-bounds)
  // weights it never uses, as it did before with the last slot's
  weights(min(wave, a.E - 1), bw0, sc0);
  __builtin_amdgcn_sched_barrier(0);
  slot_pos[tid] = spos;  // entries past R are not read
  wts[tid] = round_bf16(wrt);
  has_e[tid] = ex >= 0 && ex < a.E;
  if (has) {
#pragma unroll
    for (int b = 0; b < 16; ++b) xs[dc_slot(16 * st + b, R, sr)] = b < nb ? v[b] : u32x4_t{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  const ExactRegs kr = exact_regs();
  // one expert's rows times its 16 x K weight tile (in bw / sc), in 16-row
  // MFMA tiles -- more than 16 rows only when tokens route several of their
  // k slots to one expert -- the weighted rows into prod
  auto expert = [&](int u, const u32x4_t* bw, const uint32_t* sc) {
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
        for (int s2 = 0; s2 < 4; ++s2) A[s2] = xs[dc_slot(16 * tc + 4 * kb + s2, R, ar)];
        const u32x4_t w4 = bw[t];
        const bool s_ok = t_ok && 4 * t + kb < (a.K >> 5) && (!TILED || t < a.tpw);
        const ExactScale es = exact_scale(s_ok ? bf16_bits_to_f32(sc[t]) : 0.f);
        const u32x4_t bv[4] = {unpack_exact<true>(w4.x, es, kr), unpack_exact<true>(w4.y, es, kr),
                               unpack_exact<true>(w4.z, es, kr), unpack_exact<true>(w4.w, es, kr)};
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) acc = mfma16(A[s2], bv[s2], acc);
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
  if (U <= kDcWaves) {
    // at most one slot per wavefront (one token): no loads after the first
    // weights, so nothing is left in flight when the wavefront is done
    if (wave < U) expert(wave, bw0, sc0);
  } else {
    for (int u = wave; u < U; u += 2 * kDcWaves) {
      weights(min(u + kDcWaves, U - 1), bw1, sc1);
      expert(u, bw0, sc0);
      weights(min(u + 2 * kDcWaves, U - 1), bw0, sc0);
      if (u + kDcWaves < U) expert(u + kDcWaves, bw1, sc1);
    }
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

static size_t down_combine_lds(int rows) {
  return (size_t)16 * kDcTiles * rows * 16 + (size_t)rows * kDcCols * 4 + (size_t)kDcThreads * 12;
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
  const size_t lds = down_combine_lds(rows);
  if (a.wt != nullptr) {
    // the tiled copy's blocks are the 16-row column blocks, TPW <= 6 tiles
    if (a.tpw <= 0 || a.tpw > kDcTiles || a.tpw % 2 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_down_combine<true>, grid, dim3(kDcThreads), lds, s, a);
  } else {
    hipLaunchKernelGGL(k_down_combine<false>, grid, dim3(kDcThreads), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace w4a16
