// Decode-shaped W4A16 kernels for gfx950: few activation rows per weight
// matrix, so the packed weights stream from HBM once and the arithmetic runs
// on 16x16x32 bf16 MFMA tiles.
//
//   k_decode<MODE, TPW, KSPLIT, ...>   persistent workgroups stream the
//                          packed weight rows of the active experts with
//                          16-byte loads (lanes kb = 0..3 of a column read 64
//                          contiguous bytes of the row per 128-wide k tile);
//                          activations are staged once per expert in LDS.
//   MODE = dense  : y = x W^T (+bias)                (quantization.py:171-175)
//   MODE = gateup : inter = gelu(x Wg^T) * (x Wu^T)  (quantization.py:112-120)
//                   columns 0..7 of the tile are gate rows n0..n0+7 and
//                   columns 8..15 the matching up rows I+n0..I+n0+7, so the
//                   gated GELU is fused into the epilogue.
//   MODE = down   : dn[t*k+j] = inter W_d^T          (quantization.py:122-127)
//
// k_combine and k_dequant are the small helpers around it.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "route_device.hpp"

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
  const ExactRegs kr = exact_regs();
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / words;
    const int wj = (int)(i - r * words);
    const float s = bf16_bits_to_f32(scale[r * ng + (wj * 8) / G]);
    st16(out + r * K + wj * 8, unpack_exact<false>(packed[i], exact_scale(s), kr));
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
// the decode MFMA kernel (persistent weight streamer)
// ---------------------------------------------------------------------------
// Operand layout of v_mfma_f32_16x16x32_bf16 as used here: lane l supplies
// A[row l%16][8*(l/16) .. +7] and B[8*(l/16) .. +7][col l%16]; the result lane
// l holds D[4*(l/16) + r][l%16], r = 0..3.  A and B only need to agree on the
// k index carried by (l/16, element), so each lane feeds 8 consecutive k
// values of its own 32-element chunk per step (MoE down: in the order
// (0,4,1,5,2,6,3,7) in which the gate_up epilogue writes its rows).
//
// Work split: every workgroup serves exactly one active expert.  The grid
// holds the workgroups that fit on the chip at once (at least one per
// possible expert slot); with U experts active, workgroup w takes slot
// w / wps, wps = grid / U (exiting if that slot is not active), and every
// wps-th of that expert's column tiles ("items": CG groups of 16 weight
// rows).
// It stages the expert's activation rows into LDS once per pass of rb rows
// (an expert with more than rb rows makes several passes over its weights),
// then streams its items.  Inside an item, each 16-row column group's K range
// is split over KSPLIT wavefronts (wavefront ks takes the contiguous 128-wide
// k tiles ks*TPW .. ks*TPW + TPW - 1, so its back-to-back loads cover whole
// 128-byte lines of each weight row), each holding TPW tiles' weight loads
// (one 16-byte load per lane per tile) in registers.  Each weight register
// is reloaded with the next item's tile as soon as it has been unpacked, so
// weight traffic stays in flight across the MFMAs, the split-K reduction
// (through LDS) and the epilogue.
//
// LDS activation layout ("fragment order"): the 16-byte piece holding
// elements 8b..8b+7 of staged row j lives at slot
//   (16*(b/16) + 4*(b%4) + (b/4)%4) * rb + j
// i.e. grouped by (k tile, lane chunk, MFMA step), so a wavefront's
// ds_read_b128 of one MFMA step is contiguous and bank-conflict free.
// Threads per workgroup: K-split shapes run four column groups of four
// wavefronts each (sixteen wavefronts, one workgroup per CU, share one
// activation stage of up to 16 rows), the others four column groups of one
// wavefront.  With fewer items than CUs the launcher runs narrow workgroups
// instead: one column group (CG = 1), four times as many workgroups, so the
// weights spread over every CU.  Both forms read the same weight blocks:
// column block colblk's wavefront ks reads block colblk * KSPLIT + ks.
constexpr int stream_threads(int ksplit) { return ksplit == 4 ? 1024 : 256; }
// LDS bytes for staged activation rows: the K-split workgroup owns its CU's
// LDS; the others leave room for several workgroups per CU
constexpr int stage_lds_budget(int ksplit) { return ksplit == 4 ? 98304 : 49152; }
// items whose weight loads are in flight per wavefront (register sets).
// One set, refilled tile by tile while the item is multiplied, measured
// fastest: deeper rings slowed the streamer down.
constexpr int kRing = 1;

__device__ __forceinline__ int frag_slot(int b, int rb, int j) {
  return (16 * (b >> 4) + 4 * (b & 3) + ((b >> 2) & 3)) * rb + j;
}

// Every weight is dequantised exactly, bf16_RNE((u - 8) * s) (unpack_exact),
// and multiplied as a bf16 operand, as the reference's dequantise-then-matmul
// does; each lane's 32-wide chunk of a k tile has one scale.
// WIDE (group size 128, an even number of groups per row): the scales of one
// item's TPW tiles are consecutive bf16 values, fetched with one load.
// TILED (MoE): the weights come in the tiled layout written by
// k_tile_decode, where each wavefront's tile of an item is one contiguous
// KiB (lane l's 16 bytes at 16 l) instead of 16 rows x 64 bytes.
// LSCALE (tiled, group size 32 or 64): after an item's TPW tiles the copy
// holds each lane's TPW scales (one per tile: its 32-wide chunk's group),
// fetched with one load like WIDE's.
//
// SELF (gate_up, E <= kSelfMaxExperts): the launch works out its own plan
// instead of reading one, and its last workgroup writes that plan (and at
// one token the routing) for the down stage (a.route):
//   kSelfRoute  one token: the last workgroup runs the top-k + sort; every
//               other finds its own expert from the router's K-split
//               partials -- the same keys the top-k compares, ranked in
//               parallel -- as the s-th smallest selected expert for its
//               slot s (the plan's ascending order, one row per expert);
//   kSelfPlan   M * topk <= blockDim.x (the wide form) routed rows of a
//               finished top-k: every workgroup ranks the rows by expert
//               in the sort's k-major order (ballots per wavefront, the
//               wavefronts' counts in LDS), scans the counts into segment
//               offsets and 16-row slots, and takes its slot's expert,
//               segment rows and tokens; the last writes the positions,
//               offsets, descriptors and counts the sort would.
// No workgroup waits for a plan written by another launch.
constexpr int kSelfMaxExperts = 128;
constexpr int kSortWavesMax = 16;  // wavefronts of the wide form

template <int MODE, int TPW, int KSPLIT, bool LONGK, bool WIDE, bool TILED = false, bool LSCALE = false,
          int SELF = kSelfNone>
__global__ __launch_bounds__(stream_threads(KSPLIT)) __attribute__((amdgpu_waves_per_eu(TPW >= 4 ? 2 : 4, 8)))
void k_decode(DecodeArgs a) {
  constexpr int kStreamThreads = stream_threads(KSPLIT);  // the wide form
  constexpr int NWAVES = kStreamThreads / 64;
  const int CG = a.cg;  // column groups per item: 4 (wide) or 1 (narrow)
  extern __shared__ __align__(16) unsigned char smem_raw[];
  u32x4_t* __restrict__ lds_a = reinterpret_cast<u32x4_t*>(smem_raw);
  const int ntiles = ((a.K >> 5) + 3) >> 2;
  static_assert(KSPLIT == 1 || KSPLIT == 4, "the split-K epilogue gives wavefront ks output row ks");
  static_assert(!WIDE || !LONGK, "wide scale loads: one group per k tile");
  static_assert(!TILED || (!LONGK && MODE != kModeDense), "tiled expert layout");
  static_assert(!LSCALE || (TILED && WIDE), "lane scales come with the tiled copy");
  // split-K partials, double-buffered so one barrier per item suffices
  __shared__ f32x4_t red[2][KSPLIT > 1 ? NWAVES : 1][64];
  __shared__ int tok[16];

  const int tid = threadIdx.x;
  // wave-uniform values are pinned to SGPRs: branches on them must be
  // scalar, or the compiler merges in-flight load registers under exec
  // masks with copies that wait for the loads
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int cg = wave / KSPLIT;
  const int ks = wave - cg * KSPLIT;
  const int j = lane & 15;   // MFMA column (weight row in the group) / A row
  const int kb = lane >> 4;  // 32-element chunk of the 128-wide k tile

  // Staging tasks (see stage): one thread per (row, k tile), or -- without a
  // K split -- two, each taking half of the task's 16 pieces.
  constexpr int HALVES = KSPLIT != 1 ? 1 : 2;
  constexpr int PIECES = 16 / HALVES;
  // gate_up with one token: every staged row is token 0's row whatever the
  // plan holds, so each stage stages that row alone (all MFMA A rows read
  // it) and the first stage's activation loads are issued here, before the
  // plan's two dependent loads (active experts, then the descriptor), whose
  // round trips they overlap instead of following.
  const bool one_tok = MODE == kModeGateUp && a.M == 1;
  u32x4_t vpre[PIECES];
  if (one_tok) {
    const int rt = HALVES == 1 ? tid : (tid >> 1), hf = HALVES == 1 ? 0 : (tid & 1);
    if (rt < ntiles) {
      const int nb = min(16, (a.K >> 3) - 16 * rt);
#pragma unroll
      for (int b = 0; b < PIECES; ++b) vpre[b] = ld16(a.act + 128 * rt + 8 * min(PIECES * hf + b, nb - 1));
    }
  }

  // this workgroup's expert and item range.  The grid is spread over the
  // experts that are active in this batch (known only here): wps
  // workgroups each, so the chip fills whatever the routing.
  // Dense: the slots are the groups of rb rows (all of them run at once, so
  // each workgroup stages its rows once and streams its items once).
  // MoE: the active count is known only here.  The descriptor of the slot
  // this workgroup gets when u_guess slots are active (the launcher's
  // likeliest count; at one token, the count) is requested together with
  // the active count, and with the guess the launcher's slot arithmetic
  // (workgroups per slot, items per workgroup, slot = blockIdx.x * magic >>
  // 32) replaces the divisions: one scalar round trip, no division chain.
  int U = MODE == kModeDense ? (a.M + a.rb - 1) / a.rb : 1;
  int e = 0, seg0 = 0, rows = a.M;
  const int ug = a.u_guess;
  const int slot_raw = a.wps_guess > 1 ? (int)__umulhi(blockIdx.x, a.slot_magic) : (int)blockIdx.x;
  if constexpr (SELF == kSelfRoute) {
    static_assert(MODE == kModeGateUp && KSPLIT == 4, "gate_up routes, 256 threads or more");
    if (blockIdx.x == gridDim.x - 1) {
      topk_sort_small_block<kRouterMaxSplit, 2, 1>(a.route);
      return;
    }
    // keys of every expert (token 0: partial[ks][0][e], splits summed in
    // order and rounded to bf16, NaN as -inf, as load_logits does); past E, 0
    __shared__ __align__(16) uint32_t rkey[kSelfMaxExperts];
    __shared__ unsigned long long rsel[kSelfMaxExperts / 32];
    const int E = a.route.E;
    if (tid < kSelfMaxExperts) {
      uint32_t key = 0u;
      if (tid < E) {
        float pv[kRouterMaxSplit];
#pragma unroll
        for (int q = 0; q < kRouterMaxSplit; ++q) pv[q] = a.route.partial[q * E + tid];
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < kRouterMaxSplit; ++q) sum += pv[q];
        const float v = bf16_bits_to_f32(f32_to_bf16_bits(sum));
        key = topk_key(v == v ? v : -INFINITY, tid);
      }
      rkey[tid] = key;
    }
    __syncthreads();
    // rank of expert x = tid / 2 among all: lanes 2x and 2x + 1 count the
    // larger keys among experts [0, 64) and [64, 128), then add the pair
    const int x = tid >> 1, h = tid & 1;
    int above = 0;
    if (tid < 2 * kSelfMaxExperts) {
      const uint32_t kx = rkey[x];
#pragma unroll
      for (int u = 0; u < 64; u += 4) {
        const uint4 k4 = *reinterpret_cast<const uint4*>(&rkey[64 * h + u]);
        above += (k4.x > kx) + (k4.y > kx) + (k4.z > kx) + (k4.w > kx);
      }
    }
    above += __builtin_amdgcn_mov_dpp(above, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]: the pair's other half
    const bool selected = tid < 2 * kSelfMaxExperts && h == 0 && x < E && above < a.route.topk;
    const unsigned long long bal = __ballot(selected);  // wavefront w: experts 32 w + bit / 2
    if (lane == 0 && wave < kSelfMaxExperts / 32) rsel[wave] = bal;
    __syncthreads();
    // slot s: the s-th smallest selected expert (clamped for the slots past
    // the top k, which return below)
    int s_left = min(slot_raw, a.route.topk - 1), ex = 0;
#pragma unroll
    for (int w = 0; w < kSelfMaxExperts / 32; ++w) {
      unsigned long long m = rsel[w];
      const int c = __popcll(m);
      if (s_left >= 0 && s_left < c) {
        for (int i = 0; i < s_left; ++i) m &= m - 1ull;
        ex = 32 * w + (__builtin_ctzll(m) >> 1);
      }
      s_left -= c;
    }
    e = __builtin_amdgcn_readfirstlane(ex);
    U = a.route.topk;
    seg0 = slot_raw;
    rows = 1;
  }
  if constexpr (SELF == kSelfPlan) {
    // entry p = tid of the sort's k-major order (p = j M + t, routed row
    // t k + j), its expert, its rank among the entries of that expert, and
    // the experts' segment offsets and first slots
    static_assert(MODE == kModeGateUp && KSPLIT == 4, "gate_up plans, the wide form");
    __shared__ int pwc[kSortWavesMax][kSelfMaxExperts];
    __shared__ int poff[kSelfMaxExperts + 1], pslot[kSelfMaxExperts + 1];
    __shared__ int psel;
    int ep = -1, prank = 0, ptok = 0;
    const TopkSortArgs& r = a.route;
    const int E = r.E, R = r.M * r.topk;
    for (int q = tid; q < kSortWavesMax * kSelfMaxExperts; q += (int)blockDim.x) (&pwc[0][0])[q] = 0;
    int prow = 0;
    if (tid < R) {
      const int jj = (int)__umulhi((uint32_t)tid, a.plan_m_magic);
      ptok = tid - jj * r.M;
      prow = ptok * r.topk + jj;
      const int64_t ev = r.idx_out[prow];
      ep = (ev >= 0 && ev < E) ? (int)ev : -1;
    }
    __syncthreads();  // pwc cleared
    // rank among this wavefront's entries of the same expert (ballots over
    // the expert's 7 bits); the lowest such lane records the count
    const bool ok = ep >= 0;
    unsigned long long same = __ballot(ok);
#pragma unroll
    for (int b = 0; b < 7; ++b) {
      const bool bit = ok && ((ep >> b) & 1);
      const unsigned long long bb = __ballot(bit);
      same &= bit ? bb : ~bb;
    }
    const unsigned long long lt = (1ull << lane) - 1ull;
    prank = __popcll(same & lt);
    if (ok && (same & lt) == 0ull) pwc[wave][ep] = __popcll(same);
    __syncthreads();
    // wavefront 0: expert counts (lane l: experts 2 l, 2 l + 1), exclusive
    // scans of rows and of 16-row slots, in expert order as the sort's plan
    const int nw = (int)blockDim.x >> 6;
    if (wave == 0) {
      int c2[2], cs = 0, ss = 0;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int x = 2 * lane + q;
        int c = 0;
        if (x < E)
          for (int w = 0; w < nw; ++w) c += pwc[w][x];
        c2[q] = c;
        cs += c;
        ss += (c + kDecodeSlotRows - 1) / kDecodeSlotRows;
      }
      const int ci = wave_incl_scan(cs, lane), si = wave_incl_scan(ss, lane);
      int off = ci - cs, sp = si - ss;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int x = 2 * lane + q;
        if (x < E) {
          poff[x] = off;
          pslot[x] = sp;
        }
        off += c2[q];
        sp += (c2[q] + kDecodeSlotRows - 1) / kDecodeSlotRows;
      }
      if (lane == 63) {
        poff[E] = ci;
        pslot[E] = si;
      }
    }
    // the entry's rank within its expert: the earlier wavefronts' entries first
    if (ok)
      for (int w = 0; w < wave; ++w) prank += pwc[w][ep];
    __syncthreads();  // poff, pslot
    U = pslot[E];
    if (blockIdx.x == gridDim.x - 1) {
      // the plan of the sort (segment positions, offsets, one descriptor per
      // 16-row slot, the slot count; no m-tile list) for the down stage
      if (ok) r.sorted_pos[poff[ep] + prank] = prow;
      if (tid < E) {
        const int c = poff[tid + 1] - poff[tid];
        r.offsets[tid] = poff[tid];
        for (int i = 0; i < (c + kDecodeSlotRows - 1) / kDecodeSlotRows; ++i)
          *reinterpret_cast<int4*>(r.desc + 4 * (pslot[tid] + i)) = plan_desc(tid, poff[tid], c, kDecodeSlotRows, i);
      }
      if (tid == 0) {
        r.offsets[E] = poff[E];
        r.counters[0] = U;
        r.counters[1] = 0;
        r.counters[2] = 0;
        r.counters[3] = 0;
      }
      return;
    }
    if (U <= 0) return;
    // this workgroup's slot (the arithmetic below), its expert (the one whose
    // slots hold it), its 16-row chunk and the chunk's tokens, in the sort's
    // order; workgroups past the slots return below
    const int wps_p = U == ug ? a.wps_guess : max(1, min(a.n_ct, ((int)gridDim.x - 1) / U));
    const int slot_p = U == ug ? slot_raw : (int)blockIdx.x / wps_p;
    if (slot_p < U) {
      if (tid < E && pslot[tid] <= slot_p && slot_p < pslot[tid + 1]) psel = tid;
      __syncthreads();
      e = __builtin_amdgcn_readfirstlane(psel);
      const int i16 = (slot_p - pslot[e]) * kDecodeSlotRows;
      seg0 = poff[e] + i16;
      rows = min(kDecodeSlotRows, poff[e + 1] - seg0);
      if (ep == e && prank >= i16 && prank < i16 + kDecodeSlotRows) tok[prank - i16] = ptok;
    }
  } else if (MODE != kModeDense && SELF == kSelfNone) {
    const int slot_g = min(slot_raw, ug - 1);
    e = ld_uniform(a.desc, 4 * slot_g);
    seg0 = ld_uniform(a.desc, 4 * slot_g + 1);
    rows = ld_uniform(a.desc, 4 * slot_g + 2);
    U = ld_uniform(a.n_active, 0);
    asm volatile("" ::"s"(e), "s"(seg0), "s"(rows), "s"(U));  // all four in flight before the first wait
    if (U <= 0) return;
  }
  const bool guessed = U == ug;  // dense: always (u_guess is its slot count)
  const int work_grid = (int)gridDim.x - (SELF != kSelfNone ? 1 : 0);
  const int wps = guessed ? a.wps_guess : max(1, min(a.n_ct, work_grid / U));
  const int slot = guessed ? slot_raw : (int)blockIdx.x / wps;
  const int part = (int)blockIdx.x - slot * wps;
  if (slot >= U) return;  // uniform across the workgroup
  if (MODE == kModeDense) {
    seg0 = slot * a.rb;
    rows = min(a.rb, a.M - seg0);
  } else if (SELF == kSelfNone && !guessed) {
    e = ld_uniform(a.desc, 4 * slot);
    seg0 = ld_uniform(a.desc, 4 * slot + 1);
    rows = ld_uniform(a.desc, 4 * slot + 2);
  }
  // Items of this workgroup.  The expert's workgroups interleave: local
  // item c of workgroup `part` is item part + c * wps, so together they read
  // the expert's weights as one front moving through memory.  Each takes
  // its own items only (the last parts one fewer when wps does not divide
  // n_ct), rounded up to the register ring depth so it walks whole rounds;
  // items past n_ct (ring padding) compute on row 0 and store nothing.
  constexpr int RING = LONGK ? 1 : kRing;
  int per = guessed ? a.per_guess : (a.n_ct + wps - 1) / wps;
  if (part >= a.n_ct - (per - 1) * wps) per -= 1;
  per = (per + RING - 1) / RING * RING;
  if (part >= a.n_ct || rows <= 0) return;
  const int begin = 0, end_pad = per;
  auto phys = [&](int c) { return part + c * wps; };

  const int K8 = a.K >> 3;
  const int nchunks = a.K >> 5;
  const int rb = a.rb;                 // staged rows per pass, a power of two <= 16
  // A row this lane reads (rows >= rb only feed output rows that are
  // discarded; one token: the one staged row)
  const int jr_read = one_tok ? 0 : j & (rb - 1);
  const int tile0 = ks * TPW;          // this wavefront's first k tile

  // Chunks past K in the last tile read zeros from LDS (their weight operand
  // is the next row's bytes); that padding is written once here and never
  // touched by staging.  Rows past the staged ones hold stale values, which
  // only reach output rows that are not stored.
  for (int b = K8 + tid / rb; b < 16 * ntiles; b += (int)blockDim.x / rb)
    lds_a[frag_slot(b, rb, tid & (rb - 1))] = u32x4_t{0u, 0u, 0u, 0u};

  const ExactRegs kr = exact_regs();

  // weight row of this lane's MFMA column for column tile ct (gate_up: lanes
  // j < 8 take gate row n0 + j, lanes j >= 8 up row I + n0 + j - 8)
  const int jrow_g = (j & 7) + (j >= 8 ? a.I : 0);
  auto weight_row = [&](int ct, bool* ok) -> int {
    const int colblk = ct * CG + cg;
    if (MODE == kModeGateUp) {
      const int n0 = colblk * 8;
      *ok = colblk * 8 + 8 <= a.I;
      return *ok ? n0 + jrow_g : 0;
    }
    const int wrow = colblk * 16 + j;
    *ok = wrow < a.N;
    return *ok ? wrow : 0;
  };

  // The expert's weight / scale matrices as buffer descriptors (SGPRs): each
  // lane carries one byte offset per item.  Rows past the matrix read as
  // zero; chunks past the row end read the next row, harmless because their
  // activation operand is zero.
  // tiled: an expert is ct_blocks blocks of TPW KiB tiles (LSCALE: each
  // block followed by the 64 lanes x TPW scales, bf16), block
  // colblk * KSPLIT + ks holding wavefront ks's tiles of column block colblk
  constexpr int kBlockBytes = TPW * (LSCALE ? 1152 : 1024);
  const int64_t wstride = TILED ? (int64_t)a.ct_blocks * (kBlockBytes / 4) : (int64_t)a.N * K8;
  const __amdgpu_buffer_rsrc_t wsrc =
      make_rsrc(reinterpret_cast<const uint32_t*>(a.wp) + (int64_t)e * wstride, (uint32_t)wstride * 4u);
  const __amdgpu_buffer_rsrc_t ssrc = make_rsrc(a.ws + (int64_t)e * a.N * a.ng, (uint32_t)a.N * a.ng * 2u);
  struct Off {
    int woff, srow;
  };
  auto off_of = [&](int ct) -> Off {
    bool ok;
    const int wrow = weight_row(ct, &ok);
    // LSCALE: srow is the byte offset of this lane's TPW scales
    if (LSCALE) {
      const int blk = ((ct * CG + cg) * KSPLIT + ks) * kBlockBytes;
      return Off{blk + 16 * lane, blk + TPW * 1024 + lane * (TPW * 2)};
    }
    if (TILED) return Off{((ct * CG + cg) * KSPLIT + ks) * (TPW * 1024) + 16 * lane, wrow * a.ng};
    return Off{wrow * K8 * 4 + 16 * kb, wrow * a.ng};
  };
  auto scale_off = [&](const Off& o, int t) -> int { return (o.srow + ((4 * t + kb) * 32) / a.G) * 2; };

  // RING register sets of one item's weight tiles each: the loads of the
  // next RING - 1 items are in flight while one item is multiplied.
  u32x4_t bw[RING][TPW];
  // raw bf16 bits, kept 16-bit until use: widening them where the loop
  // carries them would wait for the loads (see load_batch)
  uint16_t sc[RING][TPW];
  // WIDE: the item's TPW scales as packed bf16 pairs
  constexpr int SCW = (TPW + 1) / 2;
  uint32_t scw[RING][SCW];
  auto load_scales_wide = [&](int r, const Off& o) {
    const __amdgpu_buffer_rsrc_t ssrc_w = LSCALE ? wsrc : ssrc;
    const int off = LSCALE ? o.srow : (o.srow + tile0) * 2;
    if (SCW == 3) {
      typedef __attribute__((ext_vector_type(3))) uint32_t u32x3_t;
      const u32x3_t v = __builtin_bit_cast(u32x3_t, __builtin_amdgcn_raw_buffer_load_b96(ssrc_w, off, 0, 0));
      scw[r][0] = v.x; scw[r][SCW > 1 ? 1 : 0] = v.y; scw[r][SCW > 2 ? 2 : 0] = v.z;
    } else if (SCW == 2) {
      typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;
      const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(ssrc_w, off, 0, 0));
      scw[r][0] = v.x; scw[r][SCW > 1 ? 1 : 0] = v.y;
    } else {
      scw[r][0] = __builtin_amdgcn_raw_buffer_load_b32(ssrc_w, off, 0, 0);
    }
  };

  // All loads of one batch are issued back to back; converting a scale right
  // away would make the wavefront wait for it and -- loads retiring in order --
  // for every weight load before it.
  // In the order of the refills in mma_batch (WIDE: the scales, then the
  // tiles; otherwise each tile followed by its scale): with one order on
  // every path into the item loop, the compiler's waits there count only the
  // loads an item needs first.
  auto load_batch = [&](int r, const Off& o, int tb) {
    if (WIDE) load_scales_wide(r, o);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      bw[r][i] = TILED ? buf_ld16(wsrc, tb + i < ntiles ? o.woff : 16 * lane, tb + i < ntiles ? 1024 * i : 0)
                       : buf_ld16(wsrc, o.woff + 64 * tb, 64 * i);
      if (!WIDE) sc[r][i] = buf_ld_u16(ssrc, scale_off(o, tb + i));
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Stage activation rows [mc, mc + nr) into LDS.  One task = one (row, k
  // tile): 16 pieces of 16 bytes, stored in fragment order.  `first` runs
  // right after the activation loads are issued: the first pass issues the
  // weight prologue there.  Loads complete in order, so waiting for the
  // activations then does not wait for the first items' weights (at kernel
  // start every CU requests those at once); the stage completes while they
  // stream in, and the first item's MFMAs -- and the refills for the next
  // item -- start as soon as its weights land.
  auto stage = [&](int mc, int nr, auto&& first, bool preloaded) {
    __syncthreads();  // previous readers of lds_a / tok are done
    // gate_up: token of each staged row; down: the output row t*k+j of each
    // staged row (read here once, so the epilogue issues no load: a load
    // there would wait for every weight refill issued before it).  The
    // positions are read with scalar loads, which do not wait for the
    // vector loads in flight.
    if (SELF == kSelfPlan) {
      // the tokens came with the workgroup's own plan
    } else if (MODE == kModeGateUp && a.M == 1) {
      // one token: every routed row is token 0, no position load to wait for
      if (tid < 16) tok[tid] = 0;
    } else if (MODE != kModeDense) {
      int sp[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) sp[i] = ld_uniform(a.sorted_pos, seg0 + mc + min(i, nr - 1));
      if (tid < 16) {
        int v = sp[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) v = tid == i ? sp[i] : v;
        tok[tid] = MODE == kModeGateUp ? v / a.topk : v;
      }
    }
    __syncthreads();
    // One thread per (row, k tile) task, or -- without a K split -- two,
    // each taking half of its 16 pieces.  The LDS budget keeps the task count
    // within the thread count.  Without a K split the staging registers (16
    // bytes a piece, all loads issued before any is used) next to the weight
    // prologue overflow the register budget unless the task is split; the
    // K-split shapes keep whole tasks (split, or in a task loop, the compiler
    // recomputes addresses inside their item loop instead).
    auto row_of = [&](int jr) -> int64_t {
      if (MODE == kModeGateUp) return tok[jr];
      return seg0 + mc + jr;
    };
    const int task = tid;
    const bool has = task < HALVES * nr * ntiles;  // equal for both halves
    const int hf = HALVES == 1 ? 0 : (task & 1);
    const int rt = HALVES == 1 ? task : (task >> 1);
    const int jr = rt / ntiles;
    const int t = rt - jr * ntiles;
    const int nb = min(16, K8 - 16 * t);
    u32x4_t v[PIECES];
    if (preloaded) {
#pragma unroll
      for (int b = 0; b < PIECES; ++b) v[b] = vpre[b];
    } else if (has) {
      const uint16_t* src = a.act + row_of(jr) * a.K + 128 * t;
      // pieces past the row end load the last piece again and are dropped
#pragma unroll
      for (int b = 0; b < PIECES; ++b) v[b] = ld16(src + 8 * min(PIECES * hf + b, nb - 1));
    }
    first();
    if (has) {
#pragma unroll
      for (int b = 0; b < PIECES; ++b)
        if (PIECES * hf + b < nb) lds_a[frag_slot(16 * t + PIECES * hf + b, rb, jr)] = v[b];
    }
    __syncthreads();
  };

  // One tile batch into acc.  With REFILL, each weight register is reloaded
  // from `nx` as soon as it has been unpacked, so the next loads overlap the
  // rest of this item's work without a second register set.  The reload is
  // unconditional (the caller picks the source): a conditional reload makes
  // the compiler merge old and new values with register copies, and copying
  // a register that a load is filling waits for every load in flight.
  auto mma_batch = [&](int r, int tb, f32x4_t& acc, auto refill_tag, const Off& nx) {
    constexpr bool REFILL = decltype(refill_tag)::value;
    // WIDE: this item's scales leave the registers before the refill below
    // reuses them (one load, needed by the first tile anyway)
    float sfw[TPW];
    if (WIDE) {
#pragma unroll
      for (int i = 0; i < TPW; ++i)
        sfw[i] = (i & 1) ? __uint_as_float(scw[r][i >> 1] & 0xFFFF0000u) : __uint_as_float(scw[r][i >> 1] << 16);
      if (REFILL) load_scales_wide(r, nx);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      // Tiles past K (the last wavefront's spare slots) run on the last real
      // tile's activations with a zero scale, adding exactly 0: branch-free,
      // so every weight register has one unconditional definition.
      const int t = tb + i;
      const bool t_ok = t < ntiles;
      const int tc = t_ok ? t : ntiles - 1;
      u32x4_t A[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) A[s] = lds_a[frag_slot(16 * tc + 4 * kb + s, rb, jr_read)];
      // one scale per lane chunk; chunks past K get 0
      const bool s_ok = t_ok && 4 * t + kb < nchunks;
      const float sci = !s_ok ? 0.f : (WIDE ? sfw[i] : bf16_bits_to_f32(sc[r][i]));
      // MoE down rows come in the gate_up epilogue's order (0,4,1,5,2,6,3,7):
      // the weights are unpacked in that order too
      const ExactScale es = exact_scale(sci);
      u32x4_t bv[4];
      bv[0] = unpack_exact<MODE == kModeDown>(bw[r][i].x, es, kr);
      bv[1] = unpack_exact<MODE == kModeDown>(bw[r][i].y, es, kr);
      bv[2] = unpack_exact<MODE == kModeDown>(bw[r][i].z, es, kr);
      bv[3] = unpack_exact<MODE == kModeDown>(bw[r][i].w, es, kr);
      if (REFILL) {
        // tiled: tiles past K read the expert's first KiB (cached; their
        // scale is zero)
        bw[r][i] = TILED ? buf_ld16(wsrc, t_ok ? nx.woff : 16 * lane, t_ok ? 1024 * i : 0)
                         : buf_ld16(wsrc, nx.woff + 64 * tb, 64 * i);
        if (!WIDE) sc[r][i] = buf_ld_u16(ssrc, scale_off(nx, tc));
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = mfma16(A[s], bv[s], acc);
    }
  };

  // item at ring position p of a pass (0 <= p < 2 * per): the refill of the
  // last items of a pass loads the first items again for the next pass
  auto item_at = [&](int p) -> int { return begin + (p >= per ? p - per : p); };
  // After the last pass nothing useful is refilled: every lane of those
  // loads reads the expert's first bytes (one cache line, a cache hit after
  // the first wavefront) instead of the first items again, which would
  // read TPW * 16 bytes per thread from HBM that nobody uses.
  // MoE outputs (inter or dn rows, M * topk of them) through a buffer
  // descriptor: masked lanes store past its end, where the hardware drops
  // the store.  Every wavefront then issues the same stores on every item
  // (no branch around them), so the compiler can count the memory operations
  // in flight across the item loop and waits only for the next item's first
  // weights instead of all of them.
  const __amdgpu_buffer_rsrc_t osrc =
      make_rsrc(a.out, (uint32_t)a.M * (uint32_t)a.topk * (uint32_t)(MODE == kModeGateUp ? a.I : a.N) * 2u);
  constexpr int kNoStore = 0x7FFFFFF0;
  int rbuf = 0;
  // one pass of rb staged rows over all of this workgroup's items
  auto pass = [&](int mc, int nr, bool last) {
    for (int c0 = begin; c0 < end_pad; c0 += RING) {
#pragma unroll
    for (int r = 0; r < RING; ++r) {
      const int ct = c0 + r;
      bool col_ok;
      weight_row(phys(ct), &col_ok);
      const int colblk = phys(ct) * CG + cg;
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      if (!LONGK) {
        // refill this register set with the item RING positions ahead
        // (offsets scaled by 0 or 1: a select here becomes a branch, which
        // costs the loop a register)
        const int pn = ct - begin + RING;
        const int keep = (last && pn >= per) ? 0 : 1;
        const Off nx0 = off_of(phys(item_at(pn)));
        const Off nx{nx0.woff * keep, nx0.srow * keep};
        mma_batch(r, tile0, acc, std::true_type{}, nx);
      } else {
        const Off cur = off_of(phys(ct));
        for (int tb = tile0; tb < ntiles; tb += KSPLIT * TPW) {
          load_batch(0, cur, tb);
          mma_batch(0, tb, acc, std::false_type{}, cur);
        }
      }
      // split-K reduction over the KSPLIT wavefronts of this column group:
      // wavefront ks sums output row q = ks of every lane's four (in
      // wavefront order) and finishes it, so the epilogue is shared four ways
      // wavefront ks finishes output rows qlo .. qlo + QPW - 1 of every
      // lane's four (all four without a K split): outv[qq] is row qlo + qq
      constexpr int QPW = 4 / KSPLIT;
      const int qlo = ks * QPW;
      float outv[QPW];
      if (KSPLIT > 1) {
        red[rbuf][wave][lane] = acc;
        __syncthreads();
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) {
          float sum = 0.f;
#pragma unroll
          for (int w = 0; w < KSPLIT; ++w) {
            // one float at its own LDS address (indexing the f32x4 by the
            // wavefront's row would select among the four with VALU)
            const float* rp = reinterpret_cast<const float*>(&red[rbuf][cg * KSPLIT + w][lane]);
            sum += rp[qlo + qq];
          }
          outv[qq] = sum;
        }
        rbuf ^= 1;
      } else {
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) outv[qq] = acc[qq];
      }
      // output row 4*kb + q of the MFMA tile is staged row 4*kb + q of this
      // pass; only the pass's nr rows exist.  Every wavefront stores QPW
      // values per item, none of them under a branch.
      const int ibase = mc + 4 * kb + qlo;
      const int iend = mc + nr;
      if (MODE == kModeDense) {
        const int n = colblk * 16 + j;
        const float bb = (a.bias != nullptr && col_ok) ? bf16_bits_to_f32(a.bias[n]) : 0.f;
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) {
          const int i = ibase + qq;
          if (col_ok && i < iend) a.out[(int64_t)(seg0 + i) * a.N + n] = f32_to_bf16_bits(outv[qq] + bb);
        }
      } else if (MODE == kModeGateUp) {
        // lane j (< 8) holds gate column n0+j, lane j+8 the matching up column
        const int n0 = colblk * 8;
        // intermediate rows are written in the order (0,4,1,5,2,6,3,7) per
        // 8 columns, which the down streamers' unpack pairs up for free
        const int pos = (j & 3) * 2 + ((j >> 2) & 1);
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) {
          const float up = lane_xor8(outv[qq]);
          const int i = ibase + qq;
          const float gate = round_bf16(outv[qq]);
          const float act = round_bf16(gelu_tanh_f32(gate));
          const float h = act * round_bf16(up);
          const bool ok = j < 8 && i < iend && col_ok;
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(h), osrc,
                                                ok ? ((seg0 + i) * a.I + n0 + pos) * 2 : kNoStore,
                                                0, 0);
        }
      } else {
        const int n = colblk * 16 + j;
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) {
          const int i = ibase + qq;
          const int orow = tok[i - mc];
          const bool ok = col_ok && i < iend;
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(outv[qq]), osrc,
                                                ok ? (orow * a.N + n) * 2 : kNoStore, 0, 0);
        }
      }
    }
    }
  };
  // The first pass issues the weight prologue during its staging; later
  // passes find the next items' weights in flight (the refills of a pass's
  // last items load its first items again).  (Folding the first pass into
  // the loop of the later ones was measured twice as slow at decode sizes:
  // the compiler then waits for the prologue's loads before staging.)
  stage(0, one_tok ? 1 : min(rb, rows), [&] {
    if (!LONGK) {
#pragma unroll
      for (int r = 0; r < RING; ++r) load_batch(r, off_of(phys(begin + r)), tile0);
    }
  }, one_tok);
  pass(0, min(rb, rows), rows <= rb);
  for (int mc = rb; mc < rows; mc += rb) {
    const int nr = min(rb, rows - mc);
    stage(mc, one_tok ? 1 : nr, [] {}, false);
    pass(mc, nr, mc + nr >= rows);
  }
}

// Decode launch shapes: (k tiles per wavefront, wavefronts per K range).
struct DecodeShape {
  int tpw;
  int ksplit;
};

static DecodeShape decode_shape(int K) {
  const int ntiles = ((K >> 5) + 3) >> 2;
  if (ntiles <= 2) return {2, 1};
  if (ntiles <= 4) return {4, 1};
  if (ntiles <= 6) return {6, 1};   // down, K = 704: 6 tiles, 4 column groups
  if (ntiles <= 8) return {2, 4};
  if (ntiles <= 16) return {4, 4};
  return {6, 4};                    // gate_up, K = 2816: 22 tiles over 4 wavefronts
}

// activation rows staged per LDS pass: the largest power of two <= 16 whose
// fragment-layout footprint fits the shape's LDS budget
static int stage_rows(int K, int ksplit) {
  const int ntiles = ((K >> 5) + 3) >> 2;
  const int bytes_per_row = ntiles * 16 * 16;  // fragment layout pads the last tile
  int rb = 16;
  while (rb > 1 && rb * bytes_per_row > stage_lds_budget(ksplit)) rb >>= 1;
  return rb;
}

static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// LDS bytes of one workgroup: the staged activation fragments
static size_t stream_lds(const DecodeArgs& a) {
  const int ntiles = ((a.K >> 5) + 3) >> 2;
  return (size_t)ntiles * 16 * a.rb * 16;
}

// Narrow workgroups (one column group each) when the wide form would have
// fewer than W4A16_NARROW_ITEMS_PER_CU items per CU and the narrow
// workgroups stage at most W4A16_NARROW_ROWS_PER_CU activation rows per CU
// in all (each narrow workgroup stages its own rows: a dense batch of many
// rows stays wide; a MoE slot stages its routed rows, M * top_k / slots on
// average).  Measured: dense 2816 x 2816 at M = 1 / 16 9.4 -> 6.1 / 12.0 ->
// 9.3 us, MoE decode M = 1 / 2 / 8 31.0 -> 29.4 / 38.4 -> 35.3 / 66.0 -> 63.0
// us, M = 16 unchanged; dense M = 64 narrow (8 staged rows per workgroup)
// 12.1 -> 13.9 us.
#ifndef W4A16_NARROW_ITEMS_PER_CU
#define W4A16_NARROW_ITEMS_PER_CU 8
#endif
#ifndef W4A16_NARROW_ROWS_PER_CU
#define W4A16_NARROW_ROWS_PER_CU 32
#endif

// ncolblk: column blocks of 16 weight rows per expert (gate_up: 8 gate and 8
// up rows).  a.rb holds the rows an expert can stage per pass; dense
// max_slots follows from the rows staged.
template <int MODE, int TPW, int KSPLIT, bool LONGK, bool WIDE = false, bool TILED = false, bool LSCALE = false,
          int SELF = kSelfNone>
static hipError_t launch_stream(DecodeArgs a, int ncolblk, int max_slots, hipStream_t s) {
  auto kern = k_decode<MODE, TPW, KSPLIT, LONGK, WIDE, TILED, LSCALE, SELF>;
  constexpr int kWideCg = stream_threads(KSPLIT) / 64 / KSPLIT;
  const int cus = device_cus();
  // every staging task (row, k tile; two threads each without a K split)
  // has its own thread(s)
  const int ntiles = ((a.K >> 5) + 3) >> 2;
  auto rows_for = [&](int threads) {
    int rb = a.rb;
    while (rb > 1 && (KSPLIT == 1 ? 2 : 1) * rb * ntiles > threads) rb >>= 1;
    return rb;
  };
  auto slots_for = [&](int rb) { return MODE == kModeDense ? (a.M + rb - 1) / rb : max_slots; };
  const int rb_wide = rows_for(64 * KSPLIT * kWideCg), rb_narrow = rows_for(64 * KSPLIT);
  const int64_t wide_items = (int64_t)slots_for(rb_wide) * ((ncolblk + kWideCg - 1) / kWideCg);
  const int64_t narrow_items = (int64_t)slots_for(rb_narrow) * ncolblk;
  const int64_t slot_rows =
      MODE == kModeDense ? rb_narrow
                         : std::min<int64_t>(rb_narrow, ((int64_t)a.M * a.topk + max_slots - 1) / std::max(max_slots, 1));
  const bool narrow = wide_items < (int64_t)W4A16_NARROW_ITEMS_PER_CU * cus &&
                      narrow_items * slot_rows <= (int64_t)W4A16_NARROW_ROWS_PER_CU * cus;
  a.cg = narrow ? 1 : kWideCg;
  a.rb = narrow ? rb_narrow : rb_wide;
  // kSelfPlan: one routed row per thread of the wide form, one 16-row pass
  if (SELF == kSelfPlan && (narrow || a.rb != kDecodeSlotRows || a.M < 2 ||
                            (int64_t)a.M * a.topk > 64 * KSPLIT * kWideCg))
    return hipErrorNotSupported;
  a.n_ct = (ncolblk + a.cg - 1) / a.cg;
  max_slots = slots_for(a.rb);
  const int threads = 64 * KSPLIT * a.cg;
  const size_t lds = stream_lds(a);
  // the workgroups that fit on the chip at once, at least one per possible
  // expert slot and at most one per item; the kernel spreads them over the
  // experts that turn out active (dense: the row groups)
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, lds) !=
          hipSuccess || per_cu <= 0)
    per_cu = 1;
  const int64_t resident = (int64_t)cus * per_cu;
  int64_t grid = std::min<int64_t>(resident, (int64_t)max_slots * a.n_ct);
  if (grid < max_slots) grid = max_slots;
  if (grid <= 0) return hipSuccess;
  // the kernel's slot arithmetic for max_slots active slots (MoE: the
  // likeliest count; dense: the count), so it divides only when the plan
  // differs; slot_magic = floor(2^32 / wps) + 1 gives blockIdx.x / wps
  // exactly for blockIdx.x < 2^16
  a.u_guess = std::max(max_slots, 1);
  a.wps_guess = (int)std::max<int64_t>(1, std::min<int64_t>(a.n_ct, grid / a.u_guess));
  a.slot_magic = a.wps_guess > 1 ? (uint32_t)((1ull << 32) / (uint64_t)a.wps_guess + 1ull) : 0u;
  a.per_guess = (a.n_ct + a.wps_guess - 1) / a.wps_guess;
  if (grid >= (1 << 16)) return hipErrorInvalidValue;
  // SELF: one more workgroup, the last, writes the plan
  hipLaunchKernelGGL(kern, dim3((unsigned)(grid + (SELF != kSelfNone ? 1 : 0))), dim3(threads), lds, s, a);
  return hipGetLastError();
}

template <int MODE>
static hipError_t launch_decode_mode(DecodeArgs a, int max_slots, hipStream_t s) {
  const DecodeShape sh = decode_shape(a.K);
  const int ncolblk = MODE == kModeGateUp ? a.I / 8 : (a.N + 15) / 16;
  // rows staged per pass: enough for the rows an expert can have (at most
  // the row count of the batch), capped by the LDS budget
  a.rb = stage_rows(a.K, sh.ksplit);
  int rows_cap = 1;
  while (rows_cap < a.rows_hint && rows_cap < 16) rows_cap <<= 1;
  if (a.rb > rows_cap) a.rb = rows_cap;
  const int ntiles = ((a.K >> 5) + 3) >> 2;
  // one load for an item's scales: group size 128 (one group per k tile)
  // and 4-byte aligned scale rows
  const bool wide = a.G == 128 && (a.ng % 2) == 0;
#define W4A16_DEC(T_, K_)                                                          \
  return wide ? launch_stream<MODE, T_, K_, false, true>(a, ncolblk, max_slots, s) \
              : launch_stream<MODE, T_, K_, false, false>(a, ncolblk, max_slots, s)
  if (ntiles > 24) return launch_stream<MODE, 6, 4, true>(a, ncolblk, max_slots, s);
  if (sh.ksplit == 1) {
    if (sh.tpw == 2) W4A16_DEC(2, 1);
    if (sh.tpw == 4) W4A16_DEC(4, 1);
    W4A16_DEC(6, 1);
  }
  if (sh.tpw == 2) W4A16_DEC(2, 4);
  if (sh.tpw == 4) W4A16_DEC(4, 4);
  W4A16_DEC(6, 4);
#undef W4A16_DEC
}

// the SELF launch arguments: the plan's arguments, the stage rows, the slot magic
static void self_args_into(DecodeArgs& a, const TopkSortArgs& sa, int self_mode) {
  a.route = sa;
  if (self_mode == kSelfRoute) {
    a.rb = 1;
  } else {
    a.rb = kDecodeSlotRows;
    a.plan_m_magic = (uint32_t)((1ull << 32) / (uint64_t)a.M + 1ull);
  }
}

hipError_t launch_decode(int mode, DecodeArgs a, int max_slots, hipStream_t s, const TopkSortArgs* self_args,
                         int self_mode) {
  if (max_slots <= 0) return hipSuccess;
  if (self_args != nullptr) {
    if (mode != kModeGateUp || self_args->M != a.M ||
        !decode_self_supported(self_mode, false, a.M, a.K, a.I, a.G, self_args->E, self_args->topk))
      return hipErrorNotSupported;
    self_args_into(a, *self_args, self_mode);
    if (self_mode == kSelfRoute)
      return launch_stream<kModeGateUp, 6, 4, false, true, false, false, kSelfRoute>(a, a.I / 8, max_slots, s);
    return launch_stream<kModeGateUp, 6, 4, false, true, false, false, kSelfPlan>(a, a.I / 8, max_slots, s);
  }
  // MoE outputs are addressed by 32-bit byte offsets of one buffer descriptor
  if (mode != kModeDense &&
      (int64_t)a.M * a.topk * (mode == kModeGateUp ? a.I : a.N) * 2 >= (int64_t)0x7FFFFFF0)
    return hipErrorInvalidValue;
  if (mode == kModeDense) return launch_decode_mode<kModeDense>(a, max_slots, s);
  if (mode == kModeGateUp) return launch_decode_mode<kModeGateUp>(a, max_slots, s);
  return launch_decode_mode<kModeDown>(a, max_slots, s);
}

// ---------------------------------------------------------------------------
// Tiled expert weights (a load-time copy for the decode streamer).  The
// streamer reads, per item and wavefront, TPW tiles of 16 weight rows x 64
// bytes.  The tiled copy puts each such tile in one contiguous KiB, in the
// order the streamer reads them: expert e, item ct, wavefront w form one
// block of TPW KiB tiles,
//   tile i, lane l's 16 bytes = packed row r of expert e, words
//     16 t + 4 (l / 16) + s,   s = 0..3
//   with t = KS ks + i the k tile (KS = TPW), w = KSPLIT cg + ks, j = l % 16,
//   colblk = CG ct + cg and
//     gate_up: r = 8 colblk + j % 8 (+ I for j >= 8: the matching up row),
//     down:    r = 16 colblk + j;
// words past the row's K / 8 or of rows past the matrix are zero.  With
// group size 32 or 64 each block is followed by TPW * 128 bytes of scales
// (zero past K or for rows past the matrix): lane l's TPW scales at byte
// TPW KiB + 2 TPW l, tile i's the scale of its chunk, columns
// 32 (4 t + l / 16) .. + 31.
// Supported where the streamer's shape for that K has no long-K loop (and,
// for gate_up, I is a multiple of 8); group size 128 with an even group
// count per row, or 32, or 64.
// ---------------------------------------------------------------------------
struct TiledShape {
  int tpw, ksplit, nwaves, n_ct;
  int lscale;       // group size 32 / 64: per-lane scales in the copy
  int block_bytes;  // one (item, wavefront) block
};

static bool tiled_shape(int mode, int64_t H, int64_t I, int64_t G, TiledShape* t) {
  if (H <= 0 || I <= 0 || H % 32 != 0 || I % 32 != 0) return false;
  const int64_t K = mode == kModeGateUp ? H : I;
  const DecodeShape sh = decode_shape((int)K);
  const int ntiles = (int)(((K >> 5) + 3) >> 2);
  if (ntiles > 24) return false;
  t->lscale = 0;
  if (G == 128) {
    if (((K + 127) / 128) % 2 != 0) return false;  // one wide scale load per item
  } else if (G == 32 || G == 64) {
    t->lscale = 1;
  } else {
    return false;
  }
  t->tpw = sh.tpw;
  t->ksplit = sh.ksplit;
  t->nwaves = stream_threads(sh.ksplit) / 64;
  const int cg = t->nwaves / sh.ksplit;
  const int64_t ncolblk = mode == kModeGateUp ? I / 8 : (H + 15) / 16;
  t->n_ct = (int)((ncolblk + cg - 1) / cg);
  t->block_bytes = t->tpw * (t->lscale ? 1152 : 1024);
  return true;
}

// The gate_up launch's own plan (k_decode's SELF): the gate_up streamer's
// 6-tile, 4-way-split shape with one scale load per item, E <=
// kSelfMaxExperts; kSelfRoute at one token, kSelfPlan for 2 <= M, M * topk <=
// 1024 (whether the wide form runs is the launcher's to say).
bool decode_self_supported(int self_mode, bool tiled, int64_t M, int64_t H, int64_t I, int64_t G, int64_t E,
                           int64_t topk) {
  if (E > kSelfMaxExperts || topk <= 0 || topk > E || H <= 0 || H % 32 != 0) return false;
  if (self_mode == kSelfRoute ? (M != 1 || topk > 64) : (self_mode != kSelfPlan || M < 2 || M * topk > 1024))
    return false;
  const DecodeShape sh = decode_shape((int)H);
  const int ntiles = (int)(((H >> 5) + 3) >> 2);
  if (sh.tpw != 6 || sh.ksplit != 4 || ntiles > 24) return false;
  if (tiled) {
    TiledShape t;
    return tiled_shape(kModeGateUp, H, I, G, &t) && t.tpw == 6 && t.ksplit == 4;
  }
  return G == 128 && ((H + 127) / 128) % 2 == 0;
}

size_t tiled_decode_bytes_per_expert(int mode, int64_t H, int64_t I, int64_t G) {
  TiledShape t;
  if (!tiled_shape(mode, H, I, G, &t)) return 0;
  return (size_t)t.n_ct * t.nwaves * t.block_bytes;
}

bool tiled_decode_needs_scale(int G) { return G == 32 || G == 64; }

bool tiled_decode_down_geometry(int64_t H, int64_t I, int64_t G, int* tpw, int* block_bytes, int64_t* expert_bytes) {
  TiledShape t;
  if (!tiled_shape(kModeDown, H, I, G, &t) || t.ksplit != 1) return false;
  *tpw = t.tpw;
  *block_bytes = t.block_bytes;
  *expert_bytes = (int64_t)t.n_ct * t.nwaves * t.block_bytes;
  return true;
}

// one thread per 16-byte piece of the tiled copy: TPW * 64 weight pieces,
// then (LSCALE) TPW * 8 scale pieces per block
template <int MODE>
__global__ __launch_bounds__(256) void k_tile_decode(const uint32_t* __restrict__ packed,
                                                     const uint16_t* __restrict__ scale,
                                                     uint32_t* __restrict__ tiled, int N, int K, int I, int G,
                                                     TiledShape t, int64_t pieces) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= pieces) return;
  const int per_block = t.block_bytes / 16;
  const int pi = (int)(p % per_block);
  int64_t q = p / per_block;
  const int w = (int)(q % t.nwaves);
  q /= t.nwaves;
  const int ct = (int)(q % t.n_ct);
  const int64_t e = q / t.n_ct;
  const int cg = w / t.ksplit, ks = w - cg * t.ksplit;
  const int colblk = (t.nwaves / t.ksplit) * ct + cg;
  const int K8 = K / 8;
  const int ng = (K + G - 1) / G;
  auto row_of = [&](int j, bool* ok) {
    if (MODE == kModeGateUp) {
      *ok = 8 * colblk + 8 <= I;
      return 8 * colblk + (j & 7) + (j >= 8 ? I : 0);
    }
    *ok = 16 * colblk + j < N;
    return 16 * colblk + j;
  };
  u32x4_t v = {0u, 0u, 0u, 0u};
  if (pi < t.tpw * 64) {
    const int i = pi >> 6, l = pi & 63;
    const int j = l & 15, kb = l >> 4;
    bool ok;
    const int row = row_of(j, &ok);
    const int tk = ks * t.tpw + i;  // k tile of this slot
    const uint32_t* src = packed + (e * N + row) * (int64_t)K8;
    uint32_t wd[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int word = 16 * tk + 4 * kb + s;
      wd[s] = (ok && word < K8) ? src[word] : 0u;
    }
    v = u32x4_t{wd[0], wd[1], wd[2], wd[3]};
  } else {
    // scale piece: bf16 entries 8 k .. 8 k + 7 of the block's [64 lanes][TPW]
    // scales; lane l's chunk s = l / 16 of tile i
    const int k = pi - t.tpw * 64;
    uint32_t h[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int ent = 8 * k + c;
      const int l = ent / t.tpw;
      const int j = l & 15, i = ent % t.tpw, s = l >> 4;
      bool ok;
      const int row = row_of(j, &ok);
      const int chunk = 4 * (ks * t.tpw + i) + s;
      const int g = (chunk * 32) / G;
      h[c] = (ok && chunk < K / 32) ? scale[(e * N + row) * (int64_t)ng + g] : 0u;
    }
    v = u32x4_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
  }
  *reinterpret_cast<u32x4_t*>(tiled + p * 4) = v;
}

hipError_t launch_tile_decode(int mode, const int32_t* packed, const uint16_t* scale, int E, int H, int I, int G,
                              int32_t* tiled, hipStream_t s) {
  TiledShape t;
  if (!tiled_shape(mode, H, I, G, &t)) return hipErrorInvalidValue;
  if (t.lscale && scale == nullptr) return hipErrorInvalidValue;
  const int64_t pieces = (int64_t)E * t.n_ct * t.nwaves * (t.block_bytes / 16);
  if (pieces == 0) return hipSuccess;
  const dim3 grid((unsigned)((pieces + 255) / 256));
  const uint32_t* src = reinterpret_cast<const uint32_t*>(packed);
  uint32_t* dst = reinterpret_cast<uint32_t*>(tiled);
  if (mode == kModeGateUp)
    hipLaunchKernelGGL(k_tile_decode<kModeGateUp>, grid, dim3(256), 0, s, src, scale, dst, 2 * I, H, I, G, t,
                       pieces);
  else
    hipLaunchKernelGGL(k_tile_decode<kModeDown>, grid, dim3(256), 0, s, src, scale, dst, H, I, I, G, t, pieces);
  return hipGetLastError();
}

// One tiled instantiation by scale source (group size 128: the scale tensor;
// 32 / 64: the copy).
template <int MODE, int TPW, int KSPLIT>
static hipError_t launch_stream_tiled(const TiledShape& t, DecodeArgs a, int ncolblk, int max_slots,
                                      hipStream_t s) {
  if (t.lscale) return launch_stream<MODE, TPW, KSPLIT, false, true, true, true>(a, ncolblk, max_slots, s);
  return launch_stream<MODE, TPW, KSPLIT, false, true, true>(a, ncolblk, max_slots, s);
}

// The MoE streamers on tiled weights (a.wp = the tiled copy): one scale load
// per item (group size 128 from the scale tensor, an even group count; 32 /
// 64 from the copy).
hipError_t launch_decode_tiled(int mode, DecodeArgs a, int max_slots, hipStream_t s, const TopkSortArgs* self_args,
                               int self_mode) {
  if (max_slots <= 0) return hipSuccess;
  if (self_args != nullptr && (mode != kModeGateUp || self_args->M != a.M ||
                               !decode_self_supported(self_mode, true, a.M, a.K, a.I, a.G, self_args->E,
                                                      self_args->topk)))
    return hipErrorNotSupported;
  if (mode != kModeGateUp && mode != kModeDown) return hipErrorInvalidValue;
  if ((int64_t)a.M * a.topk * (mode == kModeGateUp ? a.I : a.N) * 2 >= (int64_t)0x7FFFFFF0)
    return hipErrorInvalidValue;
  TiledShape t;
  const int64_t H = mode == kModeGateUp ? a.K : a.N;
  if (!tiled_shape(mode, H, a.I, a.G, &t)) return hipErrorInvalidValue;
  a.ct_blocks = t.n_ct * t.nwaves;
  const int ncolblk = mode == kModeGateUp ? a.I / 8 : (a.N + 15) / 16;
  a.rb = stage_rows(a.K, t.ksplit);
  int rows_cap = 1;
  while (rows_cap < a.rows_hint && rows_cap < 16) rows_cap <<= 1;
  if (a.rb > rows_cap) a.rb = rows_cap;
  if (self_args != nullptr) {
    self_args_into(a, *self_args, self_mode);
    if (self_mode == kSelfRoute)
      return t.lscale ? launch_stream<kModeGateUp, 6, 4, false, true, true, true, kSelfRoute>(a, ncolblk, max_slots, s)
                      : launch_stream<kModeGateUp, 6, 4, false, true, true, false, kSelfRoute>(a, ncolblk, max_slots, s);
    return t.lscale ? launch_stream<kModeGateUp, 6, 4, false, true, true, true, kSelfPlan>(a, ncolblk, max_slots, s)
                    : launch_stream<kModeGateUp, 6, 4, false, true, true, false, kSelfPlan>(a, ncolblk, max_slots, s);
  }
  if (mode == kModeGateUp) {
    if (t.ksplit == 4) {
      if (t.tpw == 2) return launch_stream_tiled<kModeGateUp, 2, 4>(t, a, ncolblk, max_slots, s);
      if (t.tpw == 4) return launch_stream_tiled<kModeGateUp, 4, 4>(t, a, ncolblk, max_slots, s);
      return launch_stream_tiled<kModeGateUp, 6, 4>(t, a, ncolblk, max_slots, s);
    }
    if (t.tpw == 2) return launch_stream_tiled<kModeGateUp, 2, 1>(t, a, ncolblk, max_slots, s);
    if (t.tpw == 4) return launch_stream_tiled<kModeGateUp, 4, 1>(t, a, ncolblk, max_slots, s);
    return launch_stream_tiled<kModeGateUp, 6, 1>(t, a, ncolblk, max_slots, s);
  }
  if (t.ksplit == 4) {
    if (t.tpw == 2) return launch_stream_tiled<kModeDown, 2, 4>(t, a, ncolblk, max_slots, s);
    if (t.tpw == 4) return launch_stream_tiled<kModeDown, 4, 4>(t, a, ncolblk, max_slots, s);
    return launch_stream_tiled<kModeDown, 6, 4>(t, a, ncolblk, max_slots, s);
  }
  if (t.tpw == 2) return launch_stream_tiled<kModeDown, 2, 1>(t, a, ncolblk, max_slots, s);
  if (t.tpw == 4) return launch_stream_tiled<kModeDown, 4, 1>(t, a, ncolblk, max_slots, s);
  return launch_stream_tiled<kModeDown, 6, 1>(t, a, ncolblk, max_slots, s);
}

// ---------------------------------------------------------------------------
// weighted top-k combine  (quantization.py:128-129)
// y[t] = bf16( sum_j bf16( bf16(w[t,j]) * dn[t*k+j] ) ), fp32 sum in j order.
// Slots whose expert index is outside [0, E) contribute nothing.
// one thread per (token, 8 columns)
// ---------------------------------------------------------------------------
// KMAX > 0: topk <= KMAX; every slot's index, weight and 16-byte piece is
// loaded before any is used (slots past topk load slot 0 again and are
// dropped), so a thread waits for memory once instead of twice per slot.
// KMAX == 0: any topk, one slot after the other.
template <int KMAX>
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
    const int64_t r0 = (int64_t)t * topk;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto add = [&](const u32x4_t& d, float wv) {
      const float wb = round_bf16(wv);
      const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += round_bf16(bf16_bits_to_f32(dw[q] & 0xFFFFu) * wb);
        acc[2 * q + 1] += round_bf16(bf16_bits_to_f32(dw[q] >> 16) * wb);
      }
    };
    if (KMAX > 0) {
      int64_t ex[KMAX > 0 ? KMAX : 1];
      float wv[KMAX > 0 ? KMAX : 1];
      u32x4_t d[KMAX > 0 ? KMAX : 1];
#pragma unroll
      for (int jj = 0; jj < KMAX; ++jj) {
        const int64_t r = r0 + (jj < topk ? jj : 0);
        ex[jj] = idx[r];
        wv[jj] = w[r];
        d[jj] = ld16(dn + r * H + c8);
      }
#pragma unroll
      for (int jj = 0; jj < KMAX; ++jj)
        if (jj < topk && ex[jj] >= 0 && ex[jj] < E) add(d[jj], wv[jj]);
    } else {
      for (int jj = 0; jj < topk; ++jj) {
        const int64_t ex = idx[r0 + jj];
        if (ex < 0 || ex >= E) continue;
        add(ld16(dn + (r0 + jj) * H + c8), w[r0 + jj]);
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
  if (topk <= 8)
    hipLaunchKernelGGL(k_combine<8>, dim3((unsigned)blocks), dim3(256), 0, s, dn, idx, w, out, M,
                       topk, E, H);
  else
    hipLaunchKernelGGL(k_combine<0>, dim3((unsigned)blocks), dim3(256), 0, s, dn, idx, w, out, M,
                       topk, E, H);
  return hipGetLastError();
}

}  // namespace w4a16
