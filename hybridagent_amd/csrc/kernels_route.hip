// Routing kernels for gfx950:
//   k_router_norm    r = bf16(bf16(rms_norm(h) * scale) * scalar_root)   (backends.py:112)
//   k_router_logits  partial fp32 logits r @ W_r^T on 16x16x32 bf16 MFMA,
//                    split over K so a handful of tokens still fills the chip
//   k_router_topk    sum the K-splits, round to bf16 (the reference's bf16
//                    F.linear output, backends.py:113), softmax in fp32,
//                    top-k (value descending, then lower index), renormalise,
//                    multiply by per_expert_scale  (backends.py:114-117)
//   k_moe_sort       stable counting sort of the k-major flattening of
//                    top_k_index by expert -> per-expert segments in the
//                    reference's visiting order (quantization.py:266-276),
//                    plus one work descriptor per active expert and the
//                    prefill tile list (k_sort_hist + k_sort_scatter: the
//                    same over several workgroups)
//   large batches    k_router_inv + k_router_tok (the norm folded into the
//                    logits kernel's A operand)
//   decode sizes     k_router_norm_logits (norm + logits in one launch),
//                    k_router_topk_sort_small (top-k + sort in one launch)
#include "common.hpp"
#include "launch.hpp"
#include "linear_bf16.hpp"
#include "route_device.hpp"

namespace w4a16 {

// ---------------------------------------------------------------------------
// wave / block reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_f32(v); }

// ---------------------------------------------------------------------------
// router RMSNorm + scales: one workgroup (256 threads) per token row
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_router_norm(const uint16_t* __restrict__ h,
                                                     const uint16_t* __restrict__ scale,
                                                     float scalar_root, float eps,
                                                     uint16_t* __restrict__ r, int H) {
  // one pass: each thread keeps its 16-byte chunks (up to kNormChunks) in
  // registers between the sum of squares and the scaled write
  constexpr int kNormChunks = 4;  // H <= 256 * 8 * 4 = 8192 in one pass
  const int64_t row = blockIdx.x;
  const uint16_t* hr = h + row * H;
  const int n8 = H >> 3;
  __shared__ float part[4];
  u32x4_t v[kNormChunks];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = threadIdx.x + 256 * q;
    v[q] = c8 < n8 ? ld16(hr + 8 * c8) : u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const uint32_t w4[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float lo = bf16_bits_to_f32(w4[t] & 0xFFFFu), hi = bf16_bits_to_f32(w4[t] >> 16);
      ss = __builtin_fmaf(lo, lo, ss);
      ss = __builtin_fmaf(hi, hi, ss);
    }
  }
  // rows longer than the register pass (H > 8192): the remaining chunks
  for (int c8 = threadIdx.x + 256 * kNormChunks; c8 < n8; c8 += 256) {
    const u32x4_t x = ld16(hr + 8 * c8);
    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float lo = bf16_bits_to_f32(w4[t] & 0xFFFFu), hi = bf16_bits_to_f32(w4[t] >> 16);
      ss = __builtin_fmaf(lo, lo, ss);
      ss = __builtin_fmaf(hi, hi, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
  auto emit = [&](int c8, const u32x4_t& xv) {
    const u32x4_t sv = ld16(scale + 8 * c8);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, sw[4] = {sv.x, sv.y, sv.z, sv.w};
    uint32_t ow[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float rr[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float xe = bf16_bits_to_f32(hh ? (xw[t] >> 16) : (xw[t] & 0xFFFFu));
        const float se = bf16_bits_to_f32(hh ? (sw[t] >> 16) : (sw[t] & 0xFFFFu));
        const float a1 = round_bf16(xe * inv);
        const float a2 = round_bf16(a1 * se);
        rr[hh] = a2 * scalar_root;
      }
      ow[t] = pack_bf16x2(rr[0], rr[1]);
    }
    st16(r + row * H + 8 * c8, u32x4_t{ow[0], ow[1], ow[2], ow[3]});
  };
#pragma unroll
  for (int q = 0; q < kNormChunks; ++q) {
    const int c8 = threadIdx.x + 256 * q;
    if (c8 < n8) emit(c8, v[q]);
  }
  for (int c8 = threadIdx.x + 256 * kNormChunks; c8 < n8; c8 += 256) emit(c8, ld16(hr + 8 * c8));
}

hipError_t launch_router_norm(const uint16_t* h, const uint16_t* scale, float scalar_root,
                              float eps, uint16_t* r, int M, int H, hipStream_t s) {
  if (M == 0) return hipSuccess;
  hipLaunchKernelGGL(k_router_norm, dim3(M), dim3(256), 0, s, h, scale, scalar_root, eps, r, H);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// router logits: one wavefront per (16 tokens, 16 experts, K split)
// partial[ks][m][e] = sum over the split's k of r[m,k] * W_r[e,k]   (fp32)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_router_logits(const uint16_t* __restrict__ r,
                                                      const uint16_t* __restrict__ proj,
                                                      float* __restrict__ partial, int M, int H,
                                                      int E, int kchunks_per_split) {
  const int lane = threadIdx.x;
  const int j = lane & 15, kb = lane >> 4;
  const int e = blockIdx.y * 16 + j;
  const int ks = blockIdx.z;
  const int m = blockIdx.x * 16 + j;
  const int nchunks = H >> 5;
  const int c0 = ks * kchunks_per_split;
  const int c1 = min(nchunks, c0 + kchunks_per_split);
  const bool eok = e < E, mok = m < M;
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  // each MFMA step consumes 32 k: lane kb supplies k = 32c + 8kb .. +7
  for (int c = c0; c < c1; ++c) {
    const int k0 = 32 * c + 8 * kb;
    const u32x4_t av = mok ? ld16(r + (int64_t)m * H + k0) : zero4;
    const u32x4_t bv = eok ? ld16(proj + (int64_t)e * H + k0) : zero4;
    acc = mfma16(av, bv, acc);
  }
  // D lane l: rows 4*(l/16)+q (tokens), column l%16 (experts)
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int mm = blockIdx.x * 16 + 4 * kb + q;
    if (mm < M && eok) partial[((int64_t)ks * M + mm) * E + e] = acc[q];
  }
}

hipError_t launch_router_logits(const uint16_t* r, const uint16_t* proj, float* partial, int M,
                                int H, int E, int ksplit, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const int nchunks = H >> 5;
  const int per = (nchunks + ksplit - 1) / ksplit;
  dim3 grid((M + 15) / 16, (E + 15) / 16, ksplit);
  hipLaunchKernelGGL(k_router_logits, grid, dim3(64), 0, s, r, proj, partial, M, H, E, per);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// router RMSNorm + logits in one launch (decode sizes): one workgroup per
// (16 tokens, K split) covers all experts, so the norm of its rows is computed
// once per 128 experts.  Phase 1 sums x^2 over whole rows (fixed order: 32
// threads per row, each over a strided set of 16-byte chunks, then the 32
// partials in thread order); phase 2 forms r = bf16(bf16(bf16(x * inv) *
// scale) * root) for the split's k range only, straight into LDS in MFMA
// A-operand order; phase 3 is 16x16x32 MFMA against the router weights,
// whose loads are issued right after the rows' and overlap phases 1-2.
// ---------------------------------------------------------------------------
constexpr int kFusedLogitsThreads = 512;
constexpr int kFusedLogitsMaxSteps = 12;  // 32-wide k steps per split

struct RouterNormLogitsArgs {
  const uint16_t* h;
  const uint16_t* scale;
  float scalar_root, eps;
  const uint16_t* proj;
  float* partial;
  int M, H, E, steps_per_split;
};

// workgroup (bx: 16 tokens, by: K split) of the launch
__device__ __forceinline__ void router_norm_logits_block(const RouterNormLogitsArgs& args, int bx, int by) {
  const uint16_t* __restrict__ h = args.h;
  const uint16_t* __restrict__ scale = args.scale;
  const float scalar_root = args.scalar_root, eps = args.eps;
  const uint16_t* __restrict__ proj = args.proj;
  float* __restrict__ partial = args.partial;
  const int M = args.M, H = args.H, E = args.E, steps_per_split = args.steps_per_split;
  constexpr int NW = kFusedLogitsThreads / 64;
  __shared__ u32x4_t afrag[kFusedLogitsMaxSteps][64];
  __shared__ float s_part[16][33];
  __shared__ float s_inv[16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kb = lane >> 4;
  const int m0 = bx * 16;
  const int ks = by;
  const int nchunks = H >> 5;
  const int c0 = ks * steps_per_split;
  const int nsteps = max(0, min(nchunks, c0 + steps_per_split) - c0);

  u32x4_t bv[kFusedLogitsMaxSteps];

  // phase 2's activation and scale pieces, loaded now so they arrive with
  // phase 1's (one memory round trip instead of two); rows past M are
  // clamped and masked in phase 2
  constexpr int kP2 = (kFusedLogitsMaxSteps * 64 + kFusedLogitsThreads - 1) / kFusedLogitsThreads;
  u32x4_t p2x[kP2], p2s[kP2];
#pragma unroll
  for (int it = 0; it < kP2; ++it) {
    const int p = min(tid + it * kFusedLogitsThreads, max(nsteps, 1) * 64 - 1);
    const int c = p >> 6, l = p & 63;
    const int cc = nsteps > 0 ? c0 + min(c, nsteps - 1) : 0;  // a chunk inside the row
    const int k0 = 32 * cc + 8 * (l >> 4);
    p2x[it] = u32x4_t{0u, 0u, 0u, 0u};
    if (m0 + (l & 15) < M) p2x[it] = ld16(h + (int64_t)(m0 + (l & 15)) * H + k0);
    p2s[it] = ld16(scale + k0);
  }

  // phase 1: sum of squares of rows m0 .. m0+15; each thread's chunks are
  // all loaded before the first is used (H <= 384 * 8 -> at most 12 chunks)
  {
    constexpr int kChunks = kFusedLogitsMaxSteps;
    const int i = tid >> 5, sub = tid & 31;
    const int m = min(m0 + i, M - 1);
    const uint16_t* row = h + (int64_t)m * H;
    const int n8 = H >> 3;
    u32x4_t v[kChunks];
#pragma unroll
    for (int q = 0; q < kChunks; ++q) v[q] = u32x4_t{0u, 0u, 0u, 0u};
    // rows past M (their sums are never used) issue no loads
    if (m0 + i < M) {
#pragma unroll
      for (int q = 0; q < kChunks; ++q) {
        const int c8 = sub + 32 * q;
        if (c8 < n8) v[q] = ld16(row + 8 * c8);
      }
    }
    // router weight fragments of this wavefront's first 16 experts, issued
    // after the rows: loads complete in order, so the sums of squares wait
    // only for the rows and the weights arrive during phase 2
    const int ec = min(wave * 16 + j, E - 1);
#pragma unroll
    for (int c = 0; c < kFusedLogitsMaxSteps; ++c)
      if (c < nsteps) bv[c] = ld16(proj + (int64_t)ec * H + 32 * (c0 + c) + 8 * kb);
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kChunks; ++q) {
      const uint32_t w4[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float lo = bf16_bits_to_f32(w4[t] & 0xFFFFu), hi = bf16_bits_to_f32(w4[t] >> 16);
        ss = __builtin_fmaf(lo, lo, ss);
        ss = __builtin_fmaf(hi, hi, ss);
      }
    }
    s_part[i][sub] = ss;
  }
  __syncthreads();
  if (tid < 16) {
    float tot = 0.f;
    for (int q = 0; q < 32; ++q) tot += s_part[tid][q];
    s_inv[tid] = 1.0f / sqrtf(tot / (float)H + eps);
  }
  __syncthreads();

  // phase 2: r for this split's k range -> afrag[step][lane(j = row, kb)]
#pragma unroll
  for (int it = 0; it < kP2; ++it) {
    const int p = tid + it * kFusedLogitsThreads;
    if (p >= nsteps * 64) break;
    const int c = p >> 6, l = p & 63;
    const int rj = l & 15;
    const int m = m0 + rj;
    u32x4_t o = {0u, 0u, 0u, 0u};
    if (m < M) {
      const u32x4_t xv = p2x[it];
      const u32x4_t sv = p2s[it];
      const float inv = s_inv[rj];
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, sw[4] = {sv.x, sv.y, sv.z, sv.w};
      uint32_t ow[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float rr[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const float xe = bf16_bits_to_f32(hh ? (xw[q] >> 16) : (xw[q] & 0xFFFFu));
          const float se = bf16_bits_to_f32(hh ? (sw[q] >> 16) : (sw[q] & 0xFFFFu));
          const float v = round_bf16(xe * inv);
          const float v2 = round_bf16(v * se);
          rr[hh] = v2 * scalar_root;
        }
        ow[q] = pack_bf16x2(rr[0], rr[1]);
      }
      o = u32x4_t{ow[0], ow[1], ow[2], ow[3]};
    }
    afrag[c][l] = o;
  }
  __syncthreads();

  // phase 3: logits of 16 tokens x 16 experts per wavefront
  for (int eb = wave; eb * 16 < E; eb += NW) {
    const int ee = eb * 16 + j;
    if (eb != wave) {
      const int eec = min(ee, E - 1);
#pragma unroll
      for (int c = 0; c < kFusedLogitsMaxSteps; ++c)
        if (c < nsteps) bv[c] = ld16(proj + (int64_t)eec * H + 32 * (c0 + c) + 8 * kb);
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kFusedLogitsMaxSteps; ++c)
      if (c < nsteps) acc = mfma16(afrag[c][lane], bv[c], acc);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int mm = m0 + 4 * kb + q;
      if (mm < M && ee < E) partial[((int64_t)ks * M + mm) * E + ee] = acc[q];
    }
  }
}

__global__ __launch_bounds__(kFusedLogitsThreads) void k_router_norm_logits(RouterNormLogitsArgs a) {
  router_norm_logits_block(a, blockIdx.x, blockIdx.y);
}

hipError_t launch_router_norm_logits(const uint16_t* h, const uint16_t* scale, float scalar_root,
                                     float eps, const uint16_t* proj, float* partial, int M,
                                     int H, int E, int ksplit, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const int nchunks = H >> 5;
  const int per = (nchunks + ksplit - 1) / ksplit;
  if (per > kFusedLogitsMaxSteps) return hipErrorInvalidValue;
  dim3 grid((M + 15) / 16, ksplit);
  hipLaunchKernelGGL(k_router_norm_logits, grid, dim3(kFusedLogitsThreads), 0, s,
                     RouterNormLogitsArgs{h, scale, scalar_root, eps, proj, partial, M, H, E, per});
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// router for large batches, two launches.
//   k_router_inv   inv[m] = 1 / sqrt(mean(h[m]^2) + eps): one wavefront per
//                  row, each lane's chunks in order, then the wave sum
//   k_router_tok   partial[ks][m][e]: wavefront w of a workgroup owns 16
//                  tokens and 128 experts over split ks's k range.
//                  r = bf16(bf16(bf16(x * inv) * scale) * root) is
//                  formed in registers as the MFMA A operand, so every
//                  element of h is read and normalised once.  The split's
//                  k range goes in chunks of 4 steps: the 128 experts'
//                  router weights (and the scales, as fp32) of a chunk sit in
//                  one of two LDS buffers, and the next chunk's loads are in
//                  flight while a chunk is multiplied (one barrier per chunk).
// Rows past M and experts past E read clamped (in-bounds) addresses; MFMA
// rows and columns are independent, so their results are simply not stored.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_router_inv(const uint16_t* __restrict__ h,
                                                    float eps, float* __restrict__ inv, int M,
                                                    int H) {
  constexpr int kChunks = 8;  // H <= 64 * 8 * 8 = 4096 in one batch of loads
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;  // uniform per wavefront
  const uint16_t* row = h + m * H;
  const int n8 = H >> 3;
  float ss = 0.f;
  for (int b = 0; b < n8; b += 64 * kChunks) {
    u32x4_t v[kChunks];
#pragma unroll
    for (int q = 0; q < kChunks; ++q) {
      const int c8 = b + lane + 64 * q;
      v[q] = c8 < n8 ? ld16(row + 8 * c8) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < kChunks; ++q) {
      const uint32_t w4[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float lo = bf16_bits_to_f32(w4[t] & 0xFFFFu), hi = bf16_bits_to_f32(w4[t] >> 16);
        ss = __builtin_fmaf(lo, lo, ss);
        ss = __builtin_fmaf(hi, hi, ss);
      }
    }
  }
  const float tot = wave_sum(ss);
  if (lane == 0) inv[m] = 1.0f / sqrtf(tot / (float)H + eps);
}

constexpr int kTokExperts = 128;  // experts per workgroup (8 MFMA column tiles)
constexpr int kTokChunk = 4;      // k steps of 32 per LDS chunk (double-buffered)
constexpr int kTokWaves = 8;      // wavefronts per workgroup, 16 tokens each
constexpr int kTokThreads = 64 * kTokWaves;
constexpr int kTokRows = 16 * kTokWaves;
constexpr int kTokNF = kTokExperts / 16;
// LDS of one chunk: weight fragments [step][column tile][lane] (16 bytes
// each), then the scales in fp32 [step][kb][8]
constexpr int kTokBSlots = kTokChunk * kTokNF * 64;
constexpr int kTokSFloats = kTokChunk * 32;

__global__ __launch_bounds__(kTokThreads) void k_router_tok(const uint16_t* __restrict__ h,
                                                            const float* __restrict__ inv,
                                                            const uint16_t* __restrict__ scale,
                                                            float scalar_root,
                                                            const uint16_t* __restrict__ proj,
                                                            float* __restrict__ partial, int M,
                                                            int H, int E, int steps_per_split) {
  constexpr int NF = kTokNF;
  static_assert(kTokThreads == kTokExperts * 4, "one staging thread per (expert, 8-wide chunk)");
  __shared__ u32x4_t sb[2][kTokBSlots];
  __shared__ __align__(16) float ssf[2][kTokSFloats];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, kb = lane >> 4;
  const int ks = blockIdx.y;
  const int mw = blockIdx.x * kTokRows + wave * 16;
  const int eg = blockIdx.z * kTokExperts;
  const int c0 = ks * steps_per_split;
  const int c1 = min(H >> 5, c0 + steps_per_split);
  const int nq = (c1 - c0 + kTokChunk - 1) / kTokChunk;  // chunks (<= 0: empty split)

  const int m = min(mw + j, M - 1);
  const uint16_t* xrow = h + (int64_t)m * H + 8 * kb;
  const float rinv = inv[m];
  // staging role: expert se, 8-wide chunk sq of each step; its LDS slot is
  // column tile se / 16, lane (se % 16) + 16 sq (a wavefront's 64 stores
  // fill one contiguous kilobyte); threads below 4 kTokChunk also bring in
  // one 8-wide scale chunk (step tid / 4, kb tid % 4) as fp32
  const int se = tid >> 2, sq = tid & 3;
  const uint16_t* wrow = proj + (int64_t)min(eg + se, E - 1) * H + 8 * sq;
  const int sslot = (se >> 4) * 64 + (se & 15) + 16 * sq;
  const int sstep = min(tid >> 2, kTokChunk - 1), skb = tid & 3;
  f32x4_t acc[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Loads of chunk q (clamped into the split, so every chunk issues the
  // same loads; a reload of the last chunk is unused): weights, scale,
  // then activations, so waiting for the weights leaves the activations in
  // flight.
  u32x4_t st[kTokChunk], scv, xv[2][kTokChunk];
  auto step_of = [&](int q, int s2) { return min(c0 + kTokChunk * q + s2, c1 - 1); };
  auto load_w = [&](int q) {
#pragma unroll
    for (int s2 = 0; s2 < kTokChunk; ++s2) st[s2] = ld16(wrow + 32 * step_of(q, s2));
    scv = ld16(scale + 32 * step_of(q, sstep) + 8 * skb);
  };
  auto load_x = [&](int q, int buf) {
#pragma unroll
    for (int s2 = 0; s2 < kTokChunk; ++s2) xv[buf][s2] = ld16(xrow + 32 * step_of(q, s2));
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int s2 = 0; s2 < kTokChunk; ++s2) sb[buf][s2 * NF * 64 + sslot] = st[s2];
    if (tid < 4 * kTokChunk) {
      const uint32_t w4[4] = {scv.x, scv.y, scv.z, scv.w};
      f32x4_t lo, hi;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        lo[2 * t] = bf16_bits_to_f32(w4[t] & 0xFFFFu);
        lo[2 * t + 1] = bf16_bits_to_f32(w4[t] >> 16);
        hi[2 * t] = bf16_bits_to_f32(w4[t + 2] & 0xFFFFu);
        hi[2 * t + 1] = bf16_bits_to_f32(w4[t + 2] >> 16);
      }
      *reinterpret_cast<f32x4_t*>(&ssf[buf][8 * tid]) = lo;
      *reinterpret_cast<f32x4_t*>(&ssf[buf][8 * tid + 4]) = hi;
    }
  };
  auto compute = [&](int q, int buf, int xb) {
    const int ns = min(kTokChunk, c1 - c0 - kTokChunk * q);
#pragma unroll
    for (int s2 = 0; s2 < kTokChunk; ++s2) {
      if (s2 < ns) {
        const f32x4_t sl = *reinterpret_cast<const f32x4_t*>(&ssf[buf][(s2 * 4 + kb) * 8]);
        const f32x4_t sh = *reinterpret_cast<const f32x4_t*>(&ssf[buf][(s2 * 4 + kb) * 8 + 4]);
        const float sf[8] = {sl[0], sl[1], sl[2], sl[3], sh[0], sh[1], sh[2], sh[3]};
        const uint32_t xw[4] = {xv[xb][s2].x, xv[xb][s2].y, xv[xb][s2].z, xv[xb][s2].w};
        uint32_t ow[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float rr[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float xe = bf16_bits_to_f32(hh ? (xw[t] >> 16) : (xw[t] & 0xFFFFu));
            const float v1 = round_bf16(xe * rinv);
            const float v2 = round_bf16(v1 * sf[2 * t + hh]);
            rr[hh] = v2 * scalar_root;
          }
          ow[t] = pack_bf16x2(rr[0], rr[1]);
        }
        const u32x4_t a = {ow[0], ow[1], ow[2], ow[3]};
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[f] = mfma16(a, sb[buf][(s2 * NF + f) * 64 + lane], acc[f]);
      }
    }
  };

  if (nq > 0) {
    load_w(0);
    load_x(0, 0);
    stage(0);
    __syncthreads();
    // chunk q: chunk q + 1's loads in flight during its multiplication, then
    // staged into the other buffer (whose last readers, chunk q - 1, all
    // passed the previous barrier); one barrier per chunk
    for (int q = 0; q < nq; q += 2) {
      load_w(q + 1);
      load_x(q + 1, 1);
      compute(q, 0, 0);
      stage(1);
      __syncthreads();
      if (q + 1 < nq) {
        load_w(q + 2);
        load_x(q + 2, 0);
        compute(q + 1, 1, 1);
        stage(0);
        __syncthreads();
      }
    }
  }
  // D lane l: rows 4*(l/16)+q (tokens), column l%16 (experts)
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int e = eg + 16 * f + j;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int mm = mw + 4 * kb + q;
      if (mm < M && e < E) partial[((int64_t)ks * M + mm) * E + e] = acc[f][q];
    }
  }
}

// K splits of the large-batch router: enough workgroups to cover the chip
// (at least 256) with 4, 8 or 16 splits
int router_tok_splits(int64_t M, int64_t E) {
  const int64_t wgs = (M + kTokRows - 1) / kTokRows * ((E + kTokExperts - 1) / kTokExperts);
  return wgs * 4 >= 256 ? 4 : wgs * 8 >= 256 ? 8 : 16;
}

hipError_t launch_router_tok(const uint16_t* h, const uint16_t* scale, float scalar_root,
                             float eps, const uint16_t* proj, float* inv, float* partial, int M,
                             int H, int E, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const int ks = router_tok_splits(M, E);
  const int nch = H >> 5;
  const int per = (nch + ks - 1) / ks;
  hipLaunchKernelGGL(k_router_inv, dim3((M + 3) / 4), dim3(256), 0, s, h, eps, inv, M, H);
  // splits whose k range is empty (per * ks > nch) still store zeros
  const dim3 grid((M + kTokRows - 1) / kTokRows, ks, (E + kTokExperts - 1) / kTokExperts);
  hipLaunchKernelGGL(k_router_tok, grid, dim3(kTokThreads), 0, s, h, inv, scale, scalar_root,
                     proj, partial, M, H, E, per);
  return hipGetLastError();
}

template <int KS, int PER>
__device__ __forceinline__ void route_token(const float* __restrict__ partial,
                                            const uint16_t* __restrict__ logits_in,
                                            const uint16_t* __restrict__ pes,
                                            uint16_t* __restrict__ logits_out, int64_t m, int M,
                                            int E, int topk, int lane, int* sel_e, float* sel_w) {
  float lg[PER];
  load_logits<KS, PER>(partial, logits_in, logits_out, m, M, E, lane, lg);
  select_topk<PER>(lg, pes, E, topk, lane, sel_e, sel_w);
}

template <int KS, int PER>
__global__ __launch_bounds__(256) void k_router_topk(const float* __restrict__ partial,
                                                     const uint16_t* __restrict__ logits_in,
                                                     const uint16_t* __restrict__ pes,
                                                     uint16_t* __restrict__ logits_out,
                                                     int64_t* __restrict__ idx_out,
                                                     float* __restrict__ w_out, int M, int E,
                                                     int topk) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;  // uniform per wavefront
  int se;
  float sw;
  route_token<KS, PER>(partial, logits_in, pes, logits_out, m, M, E, topk, lane, &se, &sw);
  if (lane < topk) {
    idx_out[m * topk + lane] = se;
    w_out[m * topk + lane] = sw;
  }
}

template <int KS>
void launch_topk_ks(const float* partial, const uint16_t* logits_in, const uint16_t* pes,
                    uint16_t* logits_out, int64_t* idx, float* w, int M, int E, int topk,
                    hipStream_t s) {
  const dim3 grid((M + 3) / 4), block(256);
  if (E <= 64)
    hipLaunchKernelGGL((k_router_topk<KS, 1>), grid, block, 0, s, partial, logits_in, pes,
                       logits_out, idx, w, M, E, topk);
  else if (E <= 128)
    hipLaunchKernelGGL((k_router_topk<KS, 2>), grid, block, 0, s, partial, logits_in, pes,
                       logits_out, idx, w, M, E, topk);
  else if (E <= 256)
    hipLaunchKernelGGL((k_router_topk<KS, 4>), grid, block, 0, s, partial, logits_in, pes,
                       logits_out, idx, w, M, E, topk);
  else
    hipLaunchKernelGGL((k_router_topk<KS, kTopkPerLane>), grid, block, 0, s, partial, logits_in,
                       pes, logits_out, idx, w, M, E, topk);
}

hipError_t launch_router_topk(const float* partial, int ksplit, const uint16_t* logits_in,
                              const uint16_t* per_expert_scale, uint16_t* logits_out,
                              int64_t* idx, float* w, int M, int E, int topk, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (partial == nullptr)
    launch_topk_ks<0>(partial, logits_in, per_expert_scale, logits_out, idx, w, M, E, topk, s);
  else if (ksplit == kRouterMaxSplit)
    launch_topk_ks<kRouterMaxSplit>(partial, logits_in, per_expert_scale, logits_out, idx, w, M,
                                    E, topk, s);
  else if (ksplit == 8)
    launch_topk_ks<8>(partial, logits_in, per_expert_scale, logits_out, idx, w, M, E, topk, s);
  else if (ksplit == 4)
    launch_topk_ks<4>(partial, logits_in, per_expert_scale, logits_out, idx, w, M, E, topk, s);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// expert sort: one workgroup of 1024 threads
//   desc[4*u .. 4*u+3] = (expert, segment start, segment rows, 0) for the u-th
//     active expert in ascending expert order
//   counters[0] = number of active experts, counters[1] = number of prefill
//     tiles, counters[2] / [3] = where the tails of at most kPrefillTinyRows
//     rows start / end in the list
//   tiles[i] = (expert << 16) | m_tile for the i-th (expert, m-tile) pair:
//     first every tile of more than BM / 2 rows, then the segment tails of at
//     most kPrefillTinyRows rows, then the other tails of at most BM / 2 rows
//     (expert order each).  Work queues hand tiles out in list order, and the
//     prefill GEMM takes the smallest tails three n-tiles at a time, which
//     makes those items longer than the other tails'.
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;

// exclusive block scan of one int per thread; returns the exclusive prefix,
// *total gets the block total.  All threads must call it.
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v, lane);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int x = lane < kSortWaves ? wsum[lane] : 0;
    x = wave_incl_scan(x, lane);
    if (lane < kSortWaves) wsum[lane] = x;
  }
  __syncthreads();
  const int res = incl - v + (wave > 0 ? wsum[wave - 1] : 0);
  *total = wsum[kSortWaves - 1];
  __syncthreads();
  return res;
}

// From the per-expert counts (thread e holds expert e's count c, e < E <= 512):
// the segment offsets, the work descriptors (plan_slots) and the m-tile
// list; written when `write` (one workgroup writes them).  Returns thread e's
// segment start.  All threads of the kSortThreads-thread workgroup call it.
__device__ __forceinline__ int write_plan(int c, int E, int32_t* __restrict__ offsets, int32_t* __restrict__ desc,
                          int32_t* __restrict__ counters, int32_t* __restrict__ tiles, int BM, int SR,
                          int* wsum, bool write) {
  const int tid = threadIdx.x;
  int tot;
  const int off = block_excl_scan(c, wsum, &tot);
  int nact;
  const int ns = plan_slots(c, SR);
  const int apos = block_excl_scan(ns, wsum, &nact);
  // BM = 0: no m-tile list (the decode streamers read none); BM is uniform,
  // so every thread takes the same branch to the scans' barriers
  const int rem = BM > 0 ? c % BM : 0;
  const int ntail = (rem > 0 && rem <= BM / 2) ? 1 : 0;
  const int ntiny = (ntail && rem <= kPrefillTinyRows) ? 1 : 0;
  const int nmid = ntail - ntiny;
  const int nbig = BM > 0 ? (c + BM - 1) / BM - ntail : 0;
  int nbig_tot = 0, nmid_tot = 0, ntiny_tot = 0, bpos = 0, mpos = 0, tpos = 0;
  if (BM > 0) {
    bpos = block_excl_scan(nbig, wsum, &nbig_tot);
    mpos = block_excl_scan(nmid, wsum, &nmid_tot);
    tpos = block_excl_scan(ntiny, wsum, &ntiny_tot);
  }
  if (write) {
    if (tid < E) offsets[tid] = off;
    if (tid == 0) {
      offsets[E] = tot;
      counters[0] = nact;
      counters[1] = nbig_tot + nmid_tot + ntiny_tot;
      counters[2] = nbig_tot;
      counters[3] = nbig_tot + ntiny_tot;
    }
    if (tid < E)
      for (int i = 0; i < ns; ++i) *reinterpret_cast<int4*>(desc + 4 * (apos + i)) = plan_desc(tid, off, c, SR, i);
    if (tid < E) {
      for (int i = 0; i < nbig; ++i) tiles[bpos + i] = (tid << 16) | i;
      if (ntiny) tiles[nbig_tot + tpos] = (tid << 16) | nbig;
      if (nmid) tiles[nbig_tot + ntiny_tot + mpos] = (tid << 16) | nbig;
    }
  }
  return off;
}

// The counting sort, run by one workgroup of kSortThreads threads; expert_of(row)
// returns the expert of row t*k+j (global memory or this workgroup's LDS).
template <typename ExpertOf>
__device__ void moe_sort_body(ExpertOf expert_of, int M, int topk, int E,
                              int32_t* __restrict__ sorted_pos, int32_t* __restrict__ offsets,
                              int32_t* __restrict__ desc, int32_t* __restrict__ counters,
                              int32_t* __restrict__ tiles, int BM, int SR) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int run[kMaxExperts];
  __shared__ int wcnt[kSortWaves][kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int total = M * topk;


  // Entry p (k-major: p = j*M + t) is routed row t*topk + j; thread tid owns
  // p = tid + kSortThreads * r.  The experts of its first kPre entries are
  // read once, all before the first is used, and serve both the count and
  // the scatter (-1: no entry or no expert).
  constexpr int kPre = 2;  // the scatter below picks pre_e[0] / pre_e[1]
  auto expert_at = [&](int p) -> int {
    const int jj = p / M, t = p - jj * M;
    const int64_t ev = expert_of(t * topk + jj);
    return (ev >= 0 && ev < E) ? (int)ev : -1;
  };
  int pre_e[kPre];
#pragma unroll
  for (int r = 0; r < kPre; ++r) {
    const int p = tid + kSortThreads * r;
    const int ev = total > 0 ? expert_at(min(p, total - 1)) : -1;
    pre_e[r] = (p < total) ? ev : -1;
  }

  for (int e = tid; e < E; e += kSortThreads) {
    cnt[e] = 0;
    for (int w = 0; w < kSortWaves; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kPre; ++r)
    if (pre_e[r] >= 0) atomicAdd(&cnt[pre_e[r]], 1);
  for (int p = tid + kSortThreads * kPre; p < total; p += kSortThreads) {
    const int e = expert_at(p);
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();

  // offsets, work descriptors, tile list and scatter bases, by wavefront 0
  if (wave == 0) plan_wave(cnt, run, E, offsets, desc, counters, tiles, BM, SR);
  __syncthreads();

  // stable scatter in k-major order p = j*M + t
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  for (int base = 0, r = 0; base < total; base += kSortThreads, ++r) {
    const int p = base + tid;
    int e = -1, row = 0;
    if (p < total) {
      const int jj = p / M, t = p - jj * M;
      row = t * topk + jj;
      e = r < kPre ? (r == 0 ? pre_e[0] : pre_e[kPre - 1]) : expert_at(p);
    }
    const bool ok = e >= 0;
    unsigned long long same = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = ok && ((e >> b) & 1);
      const unsigned long long bb = __ballot(bit);
      same &= bit ? bb : ~bb;
    }
    const int rank = __popcll(same & lt_mask);
    if (ok && (same & lt_mask) == 0ull) wcnt[wave][e] = __popcll(same);
    __syncthreads();
    if (ok) {
      int pre = run[e];
      for (int w = 0; w < wave; ++w) pre += wcnt[w][e];
      sorted_pos[pre + rank] = row;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += kSortThreads) {
      int s2 = 0;
      for (int w = 0; w < kSortWaves; ++w) {
        s2 += wcnt[w][ee];
        wcnt[w][ee] = 0;
      }
      run[ee] += s2;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kSortThreads) void k_moe_sort(
    const int64_t* __restrict__ idx_in, int M, int topk, int E, int32_t* __restrict__ sorted_pos,
    int32_t* __restrict__ offsets, int32_t* __restrict__ desc, int32_t* __restrict__ counters,
    int32_t* __restrict__ tiles, int BM, int SR, int32_t* __restrict__ queues) {
  if (queues != nullptr && threadIdx.x < kPrefillQueueInts) queues[threadIdx.x] = 0;
  moe_sort_body([&](int row) -> int64_t { return idx_in[row]; }, M, topk, E, sorted_pos, offsets,
                desc, counters, tiles, BM, SR);
}

template <int KS, int PER, int ROUNDS>
__global__ __launch_bounds__(64 * kSmallSortWaves) void k_router_topk_sort_small(TopkSortArgs a) {
  topk_sort_small_block<KS, PER, ROUNDS>(a);
}

// plan_wave's BM and slot rows: 0 or a power of two
static bool pow2_or_zero(int v) { return v >= 0 && (v & (v - 1)) == 0; }

hipError_t launch_topk_sort(const float* partial, int ksplit, const uint16_t* per_expert_scale,
                            int64_t* idx, float* w, int M, int E, int topk, int32_t* sorted_pos,
                            int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                            int BM, int slot_rows, hipStream_t s) {
  if (M == 0) return hipSuccess;
  // the decode router's partials (kRouterMaxSplit K splits), at most 64
  // routed rows: one token per wavefront up to M = 8, else eight rounds
  if (M * topk > 64 || ksplit != kRouterMaxSplit || !pow2_or_zero(BM) || !pow2_or_zero(slot_rows))
    return hipErrorInvalidValue;
  constexpr int KS = kRouterMaxSplit;
  const TopkSortArgs a{partial, per_expert_scale, idx, w, M, E, topk, sorted_pos, offsets, desc, counters, tiles, BM,
                       slot_rows};
#define W4A16_TS(P_)                                                                                      \
  if (M <= kSmallSortWaves)                                                                               \
    hipLaunchKernelGGL((k_router_topk_sort_small<KS, P_, 1>), dim3(1), dim3(64 * kSmallSortWaves), 0, s, a); \
  else                                                                                                    \
    hipLaunchKernelGGL((k_router_topk_sort_small<KS, P_, 64 / kSmallSortWaves>), dim3(1),                  \
                       dim3(64 * kSmallSortWaves), 0, s, a)
  if (E <= 64) {
    W4A16_TS(1);
  } else if (E <= 128) {
    W4A16_TS(2);
  } else if (E <= 256) {
    W4A16_TS(4);
  } else {
    W4A16_TS(kTopkPerLane);
  }
#undef W4A16_TS
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The FFN block's shared MLP (backends.py:105-108) inside the router's
// launches at decode sizes.  Its gate/up linear runs in the workgroups after
// the router logits' (both read only the block's normalised inputs), its down
// linear in the workgroups after the one-workgroup top-k + sort (the gate/up
// output is complete: it came from the previous launch).  The router chain's
// workgroups come first in the grid, so they are dispatched first; the
// linear's workgroups fill the CUs the router leaves idle.  Each workgroup
// runs one body, chosen by its index, with the same results as the separate
// kernels (k_router_norm_logits, k_router_topk_sort_small, k_linear_bf16).
// ---------------------------------------------------------------------------
static_assert(kFusedLogitsThreads == kLinThreads && 64 * kSmallSortWaves == kLinThreads,
              "one workgroup size for the fused bodies");

template <int MT>
__global__ __launch_bounds__(kLinThreads) void k_router_logits_with_linear(RouterNormLogitsArgs ra, int rgx,
                                                                         int rblocks, LinArgs la, int lgx) {
  const int b = blockIdx.x;
  if (b < rblocks) {
    router_norm_logits_block(ra, b % rgx, b / rgx);
    return;
  }
  const int l = b - rblocks;
  linear_bf16_block<MT, kLinGateUp>(la, l % lgx, l / lgx);
}

template <int PER>
__global__ __launch_bounds__(kLinThreads) void k_topk_sort_with_linear(TopkSortArgs ta, LinArgs la, int lgx) {
  if (blockIdx.x == 0) {
    topk_sort_small_block<kRouterMaxSplit, PER, 1>(ta);
    return;
  }
  const int l = blockIdx.x - 1;
  linear_bf16_block<1, kLinPlain>(la, l % lgx, l / lgx);
}

hipError_t launch_router_norm_logits_with_linear(const uint16_t* h, const uint16_t* scale, float scalar_root,
                                                 float eps, const uint16_t* proj, float* partial, int M, int H,
                                                 int E, int ksplit, const LinearCall& lin, hipStream_t s) {
  if (M == 0 || lin.M != M || lin.epi != kLinGateUp || lin.K % 32 != 0 || lin.K <= 0 || lin.N <= 0)
    return hipErrorNotSupported;
  const int nchunks = H >> 5;
  const int per = (nchunks + ksplit - 1) / ksplit;
  if (per > kFusedLogitsMaxSteps) return hipErrorNotSupported;
  const int mt = lin_row_tiles(lin.M);
  if (mt > 2) return hipErrorNotSupported;
  const RouterNormLogitsArgs ra{h, scale, scalar_root, eps, proj, partial, M, H, E, per};
  const int rgx = (M + 15) / 16, rblocks = rgx * ksplit;
  const LinArgs la = lin_args(lin.epi, lin.x, lin.W, lin.W2, lin.bias, lin.res, lin.out, lin.M, lin.N, lin.K);
  const int lgx = lin_grid_x(lin.epi, lin.N);
  const int64_t blocks = rblocks + (int64_t)lgx * lin_grid_y(lin.M);
  if (mt == 1)
    hipLaunchKernelGGL(k_router_logits_with_linear<1>, dim3((unsigned)blocks), dim3(kLinThreads), 0, s, ra, rgx,
                       rblocks, la, lgx);
  else
    hipLaunchKernelGGL(k_router_logits_with_linear<2>, dim3((unsigned)blocks), dim3(kLinThreads), 0, s, ra, rgx,
                       rblocks, la, lgx);
  return hipGetLastError();
}

hipError_t launch_topk_sort_with_linear(const float* partial, int ksplit, const uint16_t* per_expert_scale,
                                        int64_t* idx, float* w, int M, int E, int topk, int32_t* sorted_pos,
                                        int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                                        int BM, int slot_rows, const LinearCall& lin, hipStream_t s) {
  // one top-k round (a token per wavefront), at most 128 experts, and a
  // linear of at most 16 rows
  if (M == 0 || M * topk > 64 || M > kSmallSortWaves || ksplit != kRouterMaxSplit || E > 128 ||
      lin.epi != kLinPlain || lin.M <= 0 || lin.M > 16 || lin.K % 32 != 0 || lin.K <= 0 || lin.N <= 0)
    return hipErrorNotSupported;
  if (!pow2_or_zero(BM) || !pow2_or_zero(slot_rows)) return hipErrorInvalidValue;
  const TopkSortArgs ta{partial, per_expert_scale, idx, w, M, E, topk, sorted_pos, offsets, desc, counters, tiles,
                        BM, slot_rows};
  const LinArgs la = lin_args(lin.epi, lin.x, lin.W, lin.W2, lin.bias, lin.res, lin.out, lin.M, lin.N, lin.K);
  const int lgx = lin_grid_x(lin.epi, lin.N);
  const unsigned blocks = 1u + (unsigned)lgx;
  if (E <= 64)
    hipLaunchKernelGGL(k_topk_sort_with_linear<1>, dim3(blocks), dim3(kLinThreads), 0, s, ta, la, lgx);
  else
    hipLaunchKernelGGL(k_topk_sort_with_linear<2>, dim3(blocks), dim3(kLinThreads), 0, s, ta, la, lgx);
  return hipGetLastError();
}

// Large batches: the same stable sort over several workgroups, in two
// launches.  Workgroup b owns k-major positions [b*kSortThreads,
// (b+1)*kSortThreads).  k_sort_hist counts its experts; k_sort_scatter
// derives every expert's segment start and the counts of the blocks before
// its own from all blocks' histograms, then ranks its entries exactly as the
// one-workgroup sort does (stable within the block) and scatters them.
// Workgroup 0 also writes the offsets, descriptors and tile list.
__global__ __launch_bounds__(kSortThreads) void k_sort_hist(const int64_t* __restrict__ idx,
                                                           int M, int topk, int E,
                                                           int32_t* __restrict__ blockcnt) {
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kSortThreads) cnt[e] = 0;
  __syncthreads();
  const int total = M * topk;
  const int p = blockIdx.x * kSortThreads + tid;
  if (p < total) {
    const int jj = p / M, t = p - jj * M;
    const int64_t e = idx[(int64_t)t * topk + jj];
    if (e >= 0 && e < E) atomicAdd(&cnt[(int)e], 1);
  }
  __syncthreads();
  for (int e = tid; e < E; e += kSortThreads) blockcnt[(int64_t)blockIdx.x * E + e] = cnt[e];
}

__global__ __launch_bounds__(kSortThreads) void k_sort_scatter(
    const int64_t* __restrict__ idx, int M, int topk, int E, const int32_t* __restrict__ blockcnt,
    int32_t* __restrict__ sorted_pos, int32_t* __restrict__ offsets, int32_t* __restrict__ desc,
    int32_t* __restrict__ counters, int32_t* __restrict__ tiles, int BM, int SR, int32_t* __restrict__ queues) {
  __shared__ int base[kMaxExperts];
  __shared__ int wcnt[kSortWaves][kMaxExperts];
  __shared__ int wsum[kSortWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (queues != nullptr && blockIdx.x == 0 && tid < kPrefillQueueInts) queues[tid] = 0;
  const int b = blockIdx.x, nb = gridDim.x;
  // this thread's entry, loaded first so its latency overlaps the counts'
  const int total = M * topk;
  const int p = b * kSortThreads + tid;
  int e = -1, row = 0;
  int64_t ev = -1;
  if (p < total) {
    const int jj = p / M, t = p - jj * M;
    row = t * topk + jj;
    ev = idx[row];
  }
  // expert totals and the counts of the blocks before this one, 32 blocks'
  // counts per batch of loads (one memory round trip up to 32768 entries)
  int tot = 0, pre = 0;
  if (tid < E) {
    constexpr int U = 32;
    for (int q0 = 0; q0 < nb; q0 += U) {
      int cv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) cv[u] = q0 + u < nb ? blockcnt[(int64_t)(q0 + u) * E + tid] : 0;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        tot += cv[u];
        pre += q0 + u < b ? cv[u] : 0;
      }
    }
  }
  for (int x = tid; x < E; x += kSortThreads)
    for (int w = 0; w < kSortWaves; ++w) wcnt[w][x] = 0;
  const int off = write_plan(tot, E, offsets, desc, counters, tiles, BM, SR, wsum, b == 0);
  if (tid < E) base[tid] = off + pre;
  __syncthreads();
  if (ev >= 0 && ev < E) e = (int)ev;

  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  const bool ok = e >= 0;
  unsigned long long same = __ballot(ok);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool on = ok && ((e >> bit) & 1);
    const unsigned long long bb = __ballot(on);
    same &= on ? bb : ~bb;
  }
  const int rank = __popcll(same & lt_mask);
  if (ok && (same & lt_mask) == 0ull) wcnt[wave][e] = __popcll(same);
  __syncthreads();
  if (ok) {
    int q = base[e];
    for (int w = 0; w < wave; ++w) q += wcnt[w][e];
    sorted_pos[q + rank] = row;
  }
}

int sort_blocks(int64_t rows) { return (int)((rows + kSortThreads - 1) / kSortThreads); }

hipError_t launch_sort_multi(const int64_t* idx, int M, int topk, int E, int32_t* sorted_pos,
                             int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                             int32_t* blockcnt, int BM, int SR, hipStream_t s, int32_t* queues) {
  const int nb = sort_blocks((int64_t)M * topk);
  if (nb <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_sort_hist, dim3(nb), dim3(kSortThreads), 0, s, idx, M, topk, E, blockcnt);
  hipLaunchKernelGGL(k_sort_scatter, dim3(nb), dim3(kSortThreads), 0, s, idx, M, topk, E, blockcnt,
                     sorted_pos, offsets, desc, counters, tiles, BM, SR, queues);
  return hipGetLastError();
}

hipError_t launch_sort(const int64_t* idx, int M, int topk, int E, int32_t* sorted_pos,
                       int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                       int BM, int SR, hipStream_t s, int32_t* queues) {
  if (!pow2_or_zero(BM) || !pow2_or_zero(SR)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(kSortThreads), 0, s, idx, M, topk, E, sorted_pos,
                     offsets, desc, counters, tiles, BM, SR, queues);
  return hipGetLastError();
}

}  // namespace w4a16
