// Routing pieces shared by the routing kernels (kernels_route.hip) and the
// decode gate_up streamer's one-token form, which routes inside its own
// launch (kernels_decode.hip): the top-k of one token by one wavefront, the
// expert plan by one wavefront, and the one-workgroup top-k + sort.
#pragma once
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

// Inclusive prefix sum over the 64 lanes with DPP: row_shr 1, 2, 4, 8 scan
// each row of 16 lanes (lanes shifted in from outside the row add the 0
// passed as `old`); row_bcast:15 then adds row r's total to row r + 1 (rows
// 1 and 3), row_bcast:31 the total of rows 0-1 to rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v, int /*lane*/) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// ---------------------------------------------------------------------------
// softmax / top-k / renormalise: one wavefront per token, E <= 512
// ---------------------------------------------------------------------------
constexpr int kTopkPerLane = kMaxExperts / 64;
constexpr int kRouterMaxSplit = 16;

// Routing of one token by one wavefront: bf16 logits (from K-split partials
// or given), softmax denominator, top-k by (logit desc, index asc), weights.
// Lane i < topk returns selection i in *sel_e / *sel_w.
// Logits of token m, lane holding experts lane + 64 q, q < PER (PER =
// ceil(E / 64) rounded up to a power of two).  KS = number of K-split partial
// sums to add (4, 8 or kRouterMaxSplit), or 0 to read finished bf16 logits.  All
// loads are issued before any is used (addresses clamped into range,
// out-of-range values masked after); NaN becomes -inf so it never wins.
template <int KS, int PER>
__device__ __forceinline__ void load_logits(const float* __restrict__ partial,
                                            const uint16_t* __restrict__ logits_in,
                                            uint16_t* __restrict__ logits_out, int64_t m, int M,
                                            int E, int lane, float (&lg)[PER]) {
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
      lg[q] = (ok && v == v) ? v : -INFINITY;
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
}

// The top-k's order of expert e with bf16 logit lg (its exact value): the
// bf16 bits mapped to an unsigned order (-0 taken as +0, as the float
// comparison does) above the inverted index, so a larger key is a larger
// logit, or the same logit and a lower index; every key is above 0.
__device__ __forceinline__ uint32_t topk_key(float lg, int e) {
  uint32_t b = __float_as_uint(lg) >> 16;
  if (b == 0x8000u) b = 0u;
  const uint32_t mono = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return (mono << 16) | (0xFFFFu - (uint32_t)e);
}

// softmax (fp32) / top-k / renormalise / per_expert_scale of one token whose
// logits `lg` were loaded by load_logits; lane `it` < topk returns selection it.
template <int PER>
__device__ __forceinline__ void select_topk(const float (&lg)[PER], const uint16_t* __restrict__ pes, int E,
                            int topk, int lane, int* sel_e, float* sel_w) {
  const int per = (E + 63) >> 6;
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

  // top-k by (logit desc, index asc): logits are exact bf16 values, so each
  // expert gets a unique key (topk_key).  Each step takes the wavefront's
  // largest key (a DPP reduction) and clears it; selection `it` is kept by
  // lane `it` (topk <= 32 < 64).
  uint32_t key[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = lane + 64 * q;
    key[q] = (q < per && e < E) ? topk_key(lg[q], e) : 0u;
  }
  uint32_t my_key = 0u;
  for (int it = 0; it < topk; ++it) {
    uint32_t best = 0u;
#pragma unroll
    for (int q = 0; q < PER; ++q) best = key[q] > best ? key[q] : best;
    const uint32_t kmax = wave_max_u32(best);
#pragma unroll
    for (int q = 0; q < PER; ++q) key[q] = key[q] == kmax ? 0u : key[q];
    if (lane == it) my_key = kmax;
  }
  // lane it < topk decodes selection it; the probabilities of all k are
  // formed at once and summed across the lanes
  const int bi = (int)(0xFFFFu - (my_key & 0xFFFFu));
  const uint32_t mono = my_key >> 16;
  const uint32_t bb = (mono & 0x8000u) ? (mono & 0x7FFFu) : (~mono & 0xFFFFu);
  const float p = lane < topk ? expf(bf16_bits_to_f32(bb) - mx) / den : 0.f;
  const float psum = wave_sum_f32(p);
  const int ei = lane < topk ? bi : 0;
  *sel_e = ei;
  *sel_w = (lane < topk) ? (p / psum) * bf16_bits_to_f32(pes[ei]) : 0.f;
}

// Work descriptors of an expert with c rows: one, or with SR > 0 one per
// SR rows (the decode streamers' slots: an expert with more rows than one
// pass stages runs as several slots side by side instead of several passes
// in one workgroup).
__device__ __forceinline__ int plan_slots(int c, int SR) {
  return c <= 0 ? 0 : SR > 0 ? (c + SR - 1) / SR : 1;
}

// descriptor i of expert e (rows [off, off + c) of the segment order)
__device__ __forceinline__ int4 plan_desc(int e, int off, int c, int SR, int i) {
  return SR > 0 ? make_int4(e, off + i * SR, min(SR, c - i * SR), 0) : make_int4(e, off, c, 0);
}

// The plan from the per-expert counts cnt[0..E), by one wavefront (lane l
// owns the consecutive experts l*pe .. l*pe+pe-1, pe = ceil(E / 64) <= PE):
// segment starts into offsets[] and run[] (LDS), the descriptors, the m-tile
// list and the counters -- the tiles in write_plan's order except that the
// smallest tails are not listed apart (counters[2] = counters[3] =
// counters[1]) -- without
// workgroup barriers.  SR and BM are 0 or powers of two (shifts, not
// divisions: this runs on the decode layer's critical path); BM = 0 writes
// no tile list (counters[1] = 0), which the decode streamers do not read.
template <int PE = kMaxExperts / 64>
__device__ __forceinline__ void plan_wave(const int* cnt, int* run, int E, int32_t* __restrict__ offsets,
                                          int32_t* __restrict__ desc, int32_t* __restrict__ counters,
                                          int32_t* __restrict__ tiles, int BM, int SR) {
  const int lane = threadIdx.x & 63;
  const int pe = (E + 63) >> 6;
  const int srs = SR > 0 ? __builtin_ctz(SR) : 0, bms = BM > 0 ? __builtin_ctz(BM) : 0;
  auto n_slots = [&](int cc) { return cc <= 0 ? 0 : SR > 0 ? (cc + SR - 1) >> srs : 1; };
  auto n_small = [&](int cc) {
    const int rem = cc & (BM - 1);
    return (BM > 0 && rem > 0 && rem <= BM / 2) ? 1 : 0;
  };
  auto n_big = [&](int cc) { return BM > 0 ? ((cc + BM - 1) >> bms) - n_small(cc) : 0; };
  int c[PE];
  int cs = 0, as = 0, bs = 0, ss = 0;
#pragma unroll
  for (int q = 0; q < PE; ++q) {
    const int e = lane * pe + q;
    c[q] = (q < pe && e < E) ? cnt[e] : 0;
    cs += c[q];
    as += n_slots(c[q]);
    ss += n_small(c[q]);
    bs += n_big(c[q]);
  }
  const int ci = wave_incl_scan(cs, lane), ai = wave_incl_scan(as, lane);
  const int bi = wave_incl_scan(bs, lane), si = wave_incl_scan(ss, lane);
  const int nbig_tot = __builtin_amdgcn_readlane(bi, 63);
  int off = ci - cs, apos = ai - as, bpos = bi - bs, spos = nbig_tot + si - ss;
#pragma unroll
  for (int q = 0; q < PE; ++q) {
    const int e = lane * pe + q;
    if (q < pe && e < E) {
      offsets[e] = off;
      run[e] = off;
      const int ns = n_slots(c[q]);
      for (int i = 0; i < ns; ++i) *reinterpret_cast<int4*>(desc + 4 * (apos + i)) = plan_desc(e, off, c[q], SR, i);
      apos += ns;
      const int nb = n_big(c[q]);
      for (int i = 0; i < nb; ++i) tiles[bpos + i] = (e << 16) | i;
      bpos += nb;
      if (n_small(c[q])) tiles[spos++] = (e << 16) | nb;
      off += c[q];
    }
  }
  if (lane == 63) {
    offsets[E] = ci;
    counters[0] = ai;
    counters[1] = bi + si;
    counters[2] = bi + si;  // no tails listed apart
    counters[3] = bi + si;
  }
}

// Small batches (at most 64 routed rows, decode sizes): top-k of every token
// and the expert sort in one workgroup, no hand-off between workgroups.
// Eight wavefronts do the top-k (ROUNDS tokens each; the routing also lands
// in LDS), then one wavefront sorts the rows -- one row per lane: expert counts by LDS atomics, plan_wave, the stable rank among
// lower lanes of the same expert by ballots -- with no workgroup barrier
// after the top-k (a wavefront's LDS operations complete in order).
constexpr int kSmallSortWaves = 8;

template <int KS, int PER, int ROUNDS>
__device__ __forceinline__ void topk_sort_small_block(const TopkSortArgs& args) {
  const float* __restrict__ partial = args.partial;
  const uint16_t* __restrict__ pes = args.pes;
  int64_t* __restrict__ idx_out = args.idx_out;
  float* __restrict__ w_out = args.w_out;
  const int M = args.M, E = args.E, topk = args.topk, BM = args.BM;
  int32_t* __restrict__ sorted_pos = args.sorted_pos;
  int32_t* __restrict__ offsets = args.offsets;
  int32_t* __restrict__ desc = args.desc;
  int32_t* __restrict__ counters = args.counters;
  int32_t* __restrict__ tiles = args.tiles;
  __shared__ int s_idx[64];
  __shared__ uint16_t s_pes[kMaxExperts];
  __shared__ int cnt[kMaxExperts];
  __shared__ int run[kMaxExperts];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    s_pes[e] = pes[e];
    cnt[e] = 0;
  }
  float lg[ROUNDS][PER];
#pragma unroll
  for (int rr = 0; rr < ROUNDS; ++rr)
    load_logits<KS, PER>(partial, nullptr, nullptr, min(wave + kSmallSortWaves * rr, M - 1), M, E,
                         lane, lg[rr]);
  __syncthreads();  // s_pes, cnt
#pragma unroll
  for (int rr = 0; rr < ROUNDS; ++rr) {
    const int m = wave + kSmallSortWaves * rr;
    if (m >= M) break;  // uniform per wavefront
    int se;
    float sw;
    select_topk<PER>(lg[rr], s_pes, E, topk, lane, &se, &sw);
    if (lane < topk) {
      idx_out[(int64_t)m * topk + lane] = se;
      w_out[(int64_t)m * topk + lane] = sw;
      s_idx[m * topk + lane] = se;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  // lane p < M * topk holds k-major entry p = j*M + t, routed row t*topk + j
  const int total = M * topk;
  int e = -1, row = 0;
  if (lane < total) {
    const int jj = lane / M, t = lane - jj * M;
    row = t * topk + jj;
    const int ev = s_idx[row];
    if (ev >= 0 && ev < E) e = ev;
  }
  const bool ok = e >= 0;
  if (ok) atomicAdd(&cnt[e], 1);
  plan_wave<PER>(cnt, run, E, offsets, desc, counters, tiles, BM, args.slot_rows);
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  unsigned long long same = __ballot(ok);
  for (int b = 0; b < nbits; ++b) {
    const bool on = ok && ((e >> b) & 1);
    const unsigned long long bb = __ballot(on);
    same &= on ? bb : ~bb;
  }
  const int rank = __popcll(same & ((1ull << lane) - 1ull));
  if (ok) sorted_pos[run[e] + rank] = row;
}

}  // namespace w4a16
