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
//                    prefill tile list.
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

// ---------------------------------------------------------------------------
// wave / block reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_f32(v); }

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  return v;
}

// ---------------------------------------------------------------------------
// router RMSNorm + scales: one workgroup (256 threads) per token row
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_router_norm(const uint16_t* __restrict__ h,
                                                     const uint16_t* __restrict__ scale,
                                                     float scalar_root, float eps,
                                                     uint16_t* __restrict__ r, int H) {
  const int64_t row = blockIdx.x;
  const uint16_t* hr = h + row * H;
  __shared__ float part[4];
  float ss = 0.f;
  for (int c = threadIdx.x; c < H; c += 256) {
    const float v = bf16_bits_to_f32(hr[c]);
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
  for (int c = threadIdx.x; c < H; c += 256) {
    const float v = round_bf16(bf16_bits_to_f32(hr[c]) * inv);
    const float v2 = round_bf16(v * bf16_bits_to_f32(scale[c]));
    r[row * H + c] = f32_to_bf16_bits(v2 * scalar_root);
  }
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
// softmax / top-k / renormalise: one wavefront per token, E <= 512
// ---------------------------------------------------------------------------
constexpr int kTopkPerLane = kMaxExperts / 64;
constexpr int kRouterMaxSplit = 8;

// Routing of one token by one wavefront: bf16 logits (from K-split partials
// or given), softmax denominator, top-k by (logit desc, index asc), weights.
// Lane i < topk returns selection i in *sel_e / *sel_w.
// KS = number of K-split partial sums to add (1 or kRouterMaxSplit), or 0 to
// read finished bf16 logits; each lane holds experts lane + 64 q, q < PER
// (PER = ceil(E / 64) rounded up to a power of two).  Every load of the token
// is issued before any is used (addresses clamped into range, out-of-range
// values masked after).
template <int KS, int PER>
__device__ void route_token(const float* __restrict__ partial,
                            const uint16_t* __restrict__ logits_in,
                            const uint16_t* __restrict__ pes, uint16_t* __restrict__ logits_out,
                            int64_t m, int M, int E, int topk, int lane, int* sel_e,
                            float* sel_w) {
  float lg[PER];
  const int per = (E + 63) >> 6;
  if (KS > 0) {
    float pv[PER][KS > 0 ? KS : 1];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = min(lane + 64 * q, E - 1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) pv[q][ks] = partial[((int64_t)ks * M + m) * E + e];
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      // summed in split order
      float sum = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sum += pv[q][ks];
      const uint16_t b = f32_to_bf16_bits(sum);
      const int e = lane + 64 * q;
      const bool ok = q < per && e < E;
      if (ok && logits_out != nullptr) logits_out[m * E + e] = b;
      const float v = bf16_bits_to_f32(b);
      lg[q] = (ok && v == v) ? v : -INFINITY;  // NaN never wins a slot
    }
  } else {
    uint16_t lb[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) lb[q] = logits_in[m * E + min(lane + 64 * q, E - 1)];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const bool ok = q < per && lane + 64 * q < E;
      const float v = bf16_bits_to_f32(lb[q]);
      lg[q] = (ok && v == v) ? v : -INFINITY;
    }
  }
  // softmax denominator over all experts (fp32)
  float mx = -INFINITY;
#pragma unroll
  for (int q = 0; q < PER; ++q) mx = fmaxf(mx, lg[q]);
  mx = wave_max_f32(mx);
  float den = 0.f;
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (q < per && lane + 64 * q < E) den += expf(lg[q] - mx);
  den = wave_sum_f32(den);

  // top-k by (logit desc, index asc).  Logits are exact bf16 values, so each
  // expert gets a unique 32-bit key: the bf16 bits mapped to an unsigned
  // order (-0 taken as +0, as the float comparison does) above the inverted
  // index.  Each step takes the wavefront's largest key (a DPP reduction) and
  // clears it; selection `it` is kept by lane `it` (topk <= 32 < 64).
  uint32_t key[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = lane + 64 * q;
    uint32_t b = __float_as_uint(lg[q]) >> 16;
    if (b == 0x8000u) b = 0u;
    const uint32_t mono = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
    key[q] = (q < per && e < E) ? ((mono << 16) | (0xFFFFu - (uint32_t)e)) : 0u;
  }
  float my_p = 0.f;
  int my_i = 0;
  float psum = 0.f;
  for (int it = 0; it < topk; ++it) {
    uint32_t best = 0u;
#pragma unroll
    for (int q = 0; q < PER; ++q) best = key[q] > best ? key[q] : best;
    const uint32_t kmax = wave_max_u32(best);
#pragma unroll
    for (int q = 0; q < PER; ++q) key[q] = key[q] == kmax ? 0u : key[q];
    const int bi = (int)(0xFFFFu - (kmax & 0xFFFFu));
    const uint32_t mono = kmax >> 16;
    const uint32_t bb = (mono & 0x8000u) ? (mono & 0x7FFFu) : (~mono & 0xFFFFu);
    const float bv = bf16_bits_to_f32(bb);
    const float p = expf(bv - mx) / den;
    if (lane == it) {
      my_p = p;
      my_i = bi;
    }
    psum += p;
  }
  *sel_e = my_i;
  *sel_w = (lane < topk) ? (my_p / psum) * bf16_bits_to_f32(pes[my_i]) : 0.f;
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
  else if (ksplit == 1)
    launch_topk_ks<1>(partial, logits_in, per_expert_scale, logits_out, idx, w, M, E, topk, s);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// expert sort: one workgroup of 1024 threads
//   desc[4*u .. 4*u+3] = (expert, segment start, segment rows, 0) for the u-th
//     active expert in ascending expert order
//   counters[0] = number of active experts, counters[1] = number of prefill tiles
//   tiles[i] = (expert << 16) | m_tile for the i-th (expert, m-tile) pair
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;

// exclusive block scan of one int per thread; returns the exclusive prefix,
// *total gets the block total.  All threads must call it.
__device__ int block_excl_scan(int v, int* wsum, int* total) {
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

__global__ __launch_bounds__(kSortThreads) void k_moe_sort(
    const int64_t* __restrict__ idx_in, int M, int topk, int E, int32_t* __restrict__ sorted_pos,
    int32_t* __restrict__ offsets, int32_t* __restrict__ desc, int32_t* __restrict__ counters,
    int32_t* __restrict__ tiles, int BM) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int run[kMaxExperts];
  __shared__ int wcnt[kSortWaves][kMaxExperts];
  __shared__ int wsum[kSortWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int total = M * topk;

  auto expert_of = [&](int row) -> int64_t { return idx_in[row]; };

  for (int e = tid; e < E; e += kSortThreads) {
    cnt[e] = 0;
    for (int w = 0; w < kSortWaves; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
  for (int p = tid; p < total; p += kSortThreads) {
    const int64_t e = expert_of(p);
    if (e >= 0 && e < E) atomicAdd(&cnt[(int)e], 1);
  }
  __syncthreads();

  // offsets, work descriptors and tile list (E <= 512 < 1024 threads)
  const int c = tid < E ? cnt[tid] : 0;
  int tot;
  const int off = block_excl_scan(c, wsum, &tot);
  if (tid < E) {
    offsets[tid] = off;
    run[tid] = off;
  }
  if (tid == 0) offsets[E] = tot;
  int nact;
  const int apos = block_excl_scan(c > 0 ? 1 : 0, wsum, &nact);
  if (tid < E && c > 0) {
    const int4 d = make_int4(tid, off, c, 0);
    *reinterpret_cast<int4*>(desc + 4 * apos) = d;
  }
  const int nt = (c + BM - 1) / BM;
  int ntiles;
  const int tpos = block_excl_scan(nt, wsum, &ntiles);
  if (tid < E)
    for (int i = 0; i < nt; ++i) tiles[tpos + i] = (tid << 16) | i;
  if (tid == 0) {
    counters[0] = nact;
    counters[1] = ntiles;
  }
  __syncthreads();

  // stable scatter in k-major order p = j*M + t
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  for (int base = 0; base < total; base += kSortThreads) {
    const int p = base + tid;
    int e = -1, row = 0;
    if (p < total) {
      const int jj = p / M, t = p - jj * M;
      row = t * topk + jj;
      const int64_t ev = expert_of(row);
      if (ev >= 0 && ev < E) e = (int)ev;
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

hipError_t launch_sort(const int64_t* idx, int M, int topk, int E, int32_t* sorted_pos,
                       int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                       int BM, hipStream_t s) {
  hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(kSortThreads), 0, s, idx, M, topk, E, sorted_pos,
                     offsets, desc, counters, tiles, BM);
  return hipGetLastError();
}

}  // namespace w4a16
