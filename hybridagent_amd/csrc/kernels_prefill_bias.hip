// Prefill-shaped W4A16 MoE expert GEMMs in the bias form (group size a
// multiple of 128), the many-rows counterpart of the decode streamer:
//
//   MODE = gateup : inter[s] = gelu(x[tok(s)] Wg^T) * (x[tok(s)] Wu^T)
//                   (quantization.py:112-120), rows s in expert-segment order,
//                   written in bias order for the down GEMM
//   MODE = down   : dn[sorted_pos[s]] = inter[s] W_d^T   (quantization.py:122-127)
//
// Work item = (m-tile of 128 rows of one expert's segment, n-tile of 256
// weight rows; gate_up: 128 gate + the matching 128 up rows), taken from
// per-XCD work queues by a persistent grid of one 512-thread workgroup per
// CU.  Eight wavefronts (2 x 4) each own a 64 x 64 block of
// v_mfma_f32_16x16x32_bf16 accumulators (items of at most 64 rows or half
// the columns: 32 x 64, 64 x 32 or 32 x 32, so every wavefront works).  Per 128-wide k tile (one scale
// group when G = 128) the workgroup stages, with direct global -> LDS loads
// (each instruction fills 1 KiB):
//   A  activation rows (bf16, already in bias order, each tile's chunks
//      transposed) in MFMA fragment order: lane l of fragment (m-tile, step
//      s) holds row l % 16, k chunk 32 (l / 16) + 8 s -- 64 contiguous bytes
//      of each row per load -- so every fragment read is one ds_read_b128;
//   B  the packed weights, 64 bytes per weight row (16 per lane chunk,
//      XOR-swizzled by row), unpacked per wavefront with four v_and_or_b32
//      per word into (128 + u) bf16 pairs;
//   c  the rows' activation sums for the tile.
// The tables hold -136 c; the tile's first MFMAs take it as their
// accumulator input, so the MFMAs produce g = sum x (128 + u) - 136 c
// = sum x (u - 8) over the tile and the fold is one fma per accumulator
// element: acc += s g.
// A ring of three k tiles
// keeps two in flight while one is multiplied; the waits count loads (every
// wavefront issues the same ones), and the barriers wait only for LDS.
//
// The tables: gate_up reads xb / crx written by k_prefill_prep (bias-ordered
// hidden rows, tile sums); down reads the intermediate rows and the
// per-(row, 128-column block) sums the gate_up epilogue writes.
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kPbThreads = 512;
constexpr int kPbBM = kPrefillBM;           // 128 rows
constexpr int kPbBN = 256;                  // weight rows per item
constexpr int kPbMT = kPbBM / 16;           // m-tiles (16 rows) per item
constexpr int kPbAStage = kPbMT * 4 * 64;   // u32x4 slots of one A stage (32 KiB)
constexpr int kPbBStage = kPbBN * 4;        // u32x4 slots of one B stage (16 KiB, packed)
constexpr int kPbMaxNg = 24;                // scale groups per row the LDS scale image holds
static_assert(kPbBM == 128, "the wavefront layout assumes 128-row items");

// LDS / register ring of 128-wide k tiles
constexpr int kPbRing = 3;

// s_waitcnt immediate for vmcnt <= n with expcnt and lgkmcnt not waited for
// (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Workgroup barrier for LDS data only.  __syncthreads() is also a memory
// fence, which makes the compiler wait for every load in flight (vmcnt(0))
// because the direct LDS loads count there -- that would drain the stage
// ring at every barrier.  Here each wavefront waits for its own LDS writes
// (and, before calling this, for the direct loads of the stage it
// publishes), then meets the others; the "memory" clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// direct global -> LDS loads: lane l's bytes land at lds_dst + l * size
__device__ __forceinline__ void lds_dma16(const void* src, u32x4_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, int voff, u32x4_t* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds_dst, 16,
                                          voff, 0, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const float* src, float* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 4, 0, 0);
}

// position of column c (0..7 inside its 8-column block) in bias order
__device__ __forceinline__ int bias_pos(int c) { return ((c & 3) << 1) | ((c >> 2) & 1); }

}  // namespace

// ---------------------------------------------------------------------------
// hidden rows -> bias order with each 128-wide k tile's 16-byte chunks
// transposed (chunk 4 kb + s stored at 4 s + kb, so MFMA steps 2h, 2h + 1
// are 128 contiguous bytes of a row), and -136 * (the sum of each row's k
// tile) into crx[t][row].  16 lanes (one DPP row) per (row, tile); lane c
// owns chunk c.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prefill_prep(const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ xb,
                                                      float* __restrict__ crx, int M, int K,
                                                      int ldx, int nkt,
                                                      int32_t* __restrict__ queues) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid < kPrefillQueueInts) queues[gid] = 0;
  const int c = (int)(gid & 15);
  const int64_t rt = gid >> 4;
  if (rt >= (int64_t)M * nkt) return;  // whole 16-lane groups
  const int64_t row = rt / nkt;
  const int t = (int)(rt - row * nkt);
  const u32x4_t v = ld16(x + row * K + 128 * t + 8 * c);
  st16(xb + row * ldx + 128 * t + 8 * (4 * (c & 3) + (c >> 2)), to_bias_order(v));
  const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
  float sum = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) sum += bf16_bits_to_f32(w4[q] & 0xFFFFu) + bf16_bits_to_f32(w4[q] >> 16);
  sum = __uint_as_float(dpp_row_reduce(__float_as_uint(sum), [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
  if (c == 0) crx[(int64_t)t * M + row] = -136.0f * sum;
}

// the tile sums in expert-segment order: crs[t][s] = crx[t][token of row s]
// for the routed rows s < offsets[E] ([nkt][ldc], ldc >= M * topk)
__global__ __launch_bounds__(256) void k_prefill_cr_gather(const float* __restrict__ crx,
                                                           const int32_t* __restrict__ sorted_pos,
                                                           const int32_t* __restrict__ rows_total,
                                                           float* __restrict__ crs, int M, int topk,
                                                           int nkt, int ldc) {
  const int n = ld_uniform(rows_total, 0);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)n * nkt;
       i += (int64_t)gridDim.x * 256) {
    const int t = (int)(i / n);
    const int srow = (int)(i - (int64_t)t * n);
    crs[(int64_t)t * ldc + srow] = crx[(int64_t)t * M + sorted_pos[srow] / topk];
  }
}

hipError_t launch_prefill_prep(const uint16_t* x, uint16_t* xb, float* crx, int M, int K, int ldx,
                               const int32_t* sorted_pos, const int32_t* rows_total, int topk,
                               float* crs, int ldc, int32_t* queues, hipStream_t s) {
  if (K % 128 != 0 || ldx < K) return hipErrorInvalidValue;
  const int nkt = K / 128;
  int64_t threads = (int64_t)M * nkt * 16;
  if (threads < kPrefillQueueInts) threads = kPrefillQueueInts;
  hipLaunchKernelGGL(k_prefill_prep, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x,
                     xb, crx, M, K, ldx, nkt, queues);
  int64_t blocks = ((int64_t)M * topk * nkt + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_prefill_cr_gather, dim3((unsigned)blocks), dim3(256), 0, s, crx, sorted_pos,
                     rows_total, crs, M, topk, nkt, ldc);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// the grouped GEMM
// ---------------------------------------------------------------------------
// One work item of the grouped GEMM.  Wavefront (wm, wn) owns MI m-tiles of
// 16 rows (rows 16 MI wm ..) and NF blocks of 16 tile rows (output columns):
//   MI = 4, NF = 4  full item: 128 rows x 256 tile rows;
//   MI = 2          items of at most 64 rows (segment tails): all eight
//                   wavefronts work on the 64 rows, half the m-tiles each;
//   NF = 2          items with half the columns (gate_up: the last 64
//                   intermediate columns when I % 128 == 64; down: the last
//                   128 output columns when N % 256 == 128).
// With a full item's wavefront layout such items leave half the wavefronts
// idle, and a lone MFMA wavefront on a SIMD issues at half rate, so they
// would take a full item's time for half its work.  The staging (every
// wavefront's loads) is the same for every shape.
template <int MODE, int MI, int NF>
__device__ __forceinline__ void pb_item(const PrefillArgs& a, unsigned char* smem, int nt, int e,
                                        int seg0, int nrows, int* next_slot, int next) {
  u32x4_t* abuf = reinterpret_cast<u32x4_t*>(smem);                          // [kPbRing][kPbAStage]
  u32x4_t* bbuf = abuf + kPbRing * kPbAStage;                                // [kPbRing][kPbBStage]
  float* crbuf = reinterpret_cast<float*>(bbuf + kPbRing * kPbBStage);       // [kPbRing][kPbBM]
  // (crbuf has one more block: the unused correction loads of wavefronts
  // 2..7 land there)
  // the item's scales, [256 tile rows][ng] bf16 (ng even, <= kPbMaxNg)
  uint16_t* sbuf = reinterpret_cast<uint16_t*>(crbuf + (kPbRing + 1) * kPbBM);
  // loads one wavefront issues per stage (all direct LDS loads): 4 A
  // blocks, 2 B blocks, 1 correction block
  constexpr int kLoads = 7;
  constexpr int RW = 16 * MI;  // rows per wavefront

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int j = lane & 15, kb = lane >> 4;
  const int K = a.K;
  const int K8 = K >> 3;
  const int nkt = (K + 127) >> 7;
  const uint32_t kMask = opaque(0x000F000Fu), kBias = opaque(kBiasPair);

  // A rows this lane brings in for m-tile `wave`: rows 8 rh + (lane & 7)
  // of the m-tile, rh = 0, 1; rows past the segment repeat its last row
  // (their results are dropped)
  const uint16_t* arow[2];
#pragma unroll
  for (int rh = 0; rh < 2; ++rh) {
    const int r = min(16 * wave + 8 * rh + (lane & 7), nrows - 1);
    const int64_t src = MODE == kModeGateUp ? a.sorted_pos[seg0 + r] / a.topk : seg0 + r;
    arow[rh] = a.act + src * a.lda;
  }
  // correction sums (segment order, [tile][row]) this lane brings in:
  // row 64 (wave & 1) + lane for wavefronts 0, 1; the others load one
  // element (unused) so every wavefront issues the same loads
  const float* crow = a.cr + seg0 + (wave < 2 ? min(64 * (wave & 1) + lane, nrows - 1) : 0);
  // weight rows of the item's 256-row B tile: gate_up tile rows 0..127 are
  // gate rows c0.., 128..255 the matching up rows (c0 = 128 nt); down tile
  // row tr is weight row 256 nt + tr
  auto weight_row = [&](int tr) -> int {
    const int w = MODE == kModeGateUp ? (tr < 128 ? 128 * nt + tr : a.I + 128 * nt + (tr - 128))
                                      : kPbBN * nt + tr;
    return min(w, a.N - 1);
  };
  const __amdgpu_buffer_rsrc_t wsrc =
      make_rsrc(reinterpret_cast<const uint32_t*>(a.wp) + (int64_t)e * a.N * K8,
                (uint32_t)a.N * K8 * 4u);
  const __amdgpu_buffer_rsrc_t ssrc = make_rsrc(a.ws + (int64_t)e * a.N * a.ng, (uint32_t)a.N * a.ng * 2u);
  // this lane's B DMA sources: instructions q = 2 wave + h bring tile
  // slots 64 q + lane = (tile row 16 q + lane / 4, physical chunk lane & 3);
  // the chunk is XOR-swizzled with the row so fragment reads spread banks
  int bdma_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tr = 16 * (2 * wave + h) + (lane >> 2);
    const int kl = (lane & 3) ^ (tr & 3);  // logical 16-byte chunk
    bdma_off[h] = weight_row(tr) * K8 * 4 + 16 * kl;
  }
  // B tile blocks (16 rows) of this wavefront.  gate_up: gate blocks first,
  // then the matching up blocks (NF = 4: 2 wn, 2 wn + 1, 8 + 2 wn, 9 + 2 wn;
  // NF = 2: wn, 8 + wn); down: NF wn + f
  int brow[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    constexpr int H2 = NF / 2;
    const int blk = MODE == kModeGateUp ? (f < H2 ? H2 * wn + f : 8 + H2 * wn + (f - H2)) : NF * wn + f;
    brow[f] = 16 * blk + j;
  }
  // LDS slot (within an m-tile) of this lane's fragment for MFMA step s:
  // row j, chunk 4 s + kb, as the A loads place it
  int a_slot[4];
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
    const int rh = j >> 3, h = s2 >> 1, cp = 4 * (s2 & 1) + kb;
    a_slot[s2] = (2 * rh + h) * 64 + 8 * (cp ^ rh) + (j & 7);
  }
  // wavefronts whose columns lie past the matrix (last n-tile) do no MFMA
  // work and store nothing; nor do those whose rows are all padding
  const bool cols_ok = MODE == kModeGateUp ? 128 * nt + 8 * NF * (wn + 1) <= a.I
                                           : kPbBN * nt + 16 * NF * (wn + 1) <= a.N;
  const bool work = cols_ok && nrows > RW * wm;

  f32x4_t acc[MI][NF];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The loads of k tile t into ring slot r, in four parts (so they can be
  // spread between MFMA steps).  Every wavefront issues the same kLoads
  // loads in every iteration (tiles past the end load the last tile again,
  // unused), so the compiler and the waits can count them.
  //   p = 0, 1: A blocks (rh = p, h = 0, 1) = rows 8 rh .. 8 rh + 7 of
  //     m-tile `wave`, chunks 8 h .. 8 h + 7 of the tile (128 contiguous
  //     bytes per row); lane l loads row 8 rh + (l & 7), chunk
  //     8 h + ((l >> 3) ^ rh) (the XOR keeps the fragment reads of rows j
  //     and j + 8 on different banks); chunks past K (row padding) are
  //     zeroed after landing;
  //   p = 2: the wavefront's two B blocks;
  //   p = 3: the correction block.
  auto issue_part = [&](int t, int r, int p) {
    const int tt = min(t, nkt - 1);
    if (p < 2) {
      const int rh = p;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        lds_dma16(arow[rh] + 128 * tt + 8 * (8 * h + ((lane >> 3) ^ rh)),
                  abuf + r * kPbAStage + wave * 256 + (2 * rh + h) * 64);
    } else if (p == 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        lds_dma16_buf(wsrc, bdma_off[h] + 64 * tt, bbuf + r * kPbBStage + (2 * wave + h) * 64);
    } else {
      lds_dma4(crow + (int64_t)tt * a.ldc, crbuf + (wave < 2 ? r * kPbBM + 64 * wave : kPbRing * kPbBM));
    }
  };
  auto issue = [&](int t, int r) {
#pragma unroll
    for (int p = 0; p < 4; ++p) issue_part(t, r, p);
  };
  // k tile t (slot r) has landed: zero its A chunks past K (chunk c holds
  // the original k = 128 t + 32 (c % 4) + 8 (c / 4))
  auto land = [&](int t, int r) {
    if (t < nkt && 128 * t + 128 > K) {
#pragma unroll
      for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int c = 8 * h + ((lane >> 3) ^ rh);
          if (128 * t + 32 * (c & 3) + 8 * (c >> 2) >= K)
            abuf[r * kPbAStage + wave * 256 + (2 * rh + h) * 64 + lane] = u32x4_t{0u, 0u, 0u, 0u};
        }
    }
  };
  // multiply k tile t (slot r) and fold it into the accumulators; the
  // loads of tile tn (slot rn) are issued between the MFMA steps, so a
  // load that waits for a free slot in the memory pipeline delays MFMAs
  // already issued rather than the start of the tile
  auto compute = [&](int t, int r, int tn, int rn) {
    // this lane's scales (tile rows brow[f], group of k tile t)
    const int gi = (128 * t) / a.G;
    float sf[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) sf[f] = bf16_bits_to_f32(sbuf[brow[f] * a.ng + gi]);
    u32x4_t bw[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) bw[f] = bbuf[r * kPbBStage + brow[f] * 4 + (kb ^ (brow[f] & 3))];
    // -136 * the tile sums of this lane's output rows (4 kb .. 4 kb + 3 of
    // m-tile i): the accumulator input of the tile's first MFMAs
    f32x4_t ncr[MI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
      ncr[i] = *reinterpret_cast<const f32x4_t*>(crbuf + r * kPbBM + 16 * (wm * MI + i) + 4 * kb);
    f32x4_t g[MI][NF];
    // B fragments of step 0; each later step's fragment f is unpacked as
    // soon as the MI MFMAs of the current step have read fragment f, so the
    // unpack (VALU) of one column block runs beside the MFMAs of the next
    u32x4_t bv[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) bv[f] = unpack_bias(bw[f].x, kMask, kBias);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t af[MI];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = abuf[r * kPbAStage + (wm * MI + i) * 256 + a_slot[s]];
#pragma unroll
      for (int f = 0; f < NF; ++f) {
#pragma unroll
        for (int i = 0; i < MI; ++i) g[i][f] = mfma16(af[i], bv[f], s == 0 ? ncr[i] : g[i][f]);
        if (s < 3) {
          const uint32_t wd = s == 0 ? bw[f].y : s == 1 ? bw[f].z : bw[f].w;
          bv[f] = unpack_bias(wd, kMask, kBias);
        }
      }
      issue_part(tn, rn, s);
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[i][f][q] = __builtin_fmaf(sf[f], g[i][f][q], acc[i][f][q]);
  };
  // k tile t + 1 must have landed; t + 2 may still be loading
  auto wait_next = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vm_wait(kLoads));
    __builtin_amdgcn_sched_barrier(0);
  };

  lds_barrier();  // the previous item's epilogue is done with LDS
  // the item's scales: 16-byte chunks c < 32 ng of the [256][ng] image
  // (gate_up: 128 gate rows, then the 128 up rows), one 1 KiB block per
  // load, spread over the wavefronts; issued before the first tiles, so
  // the first wait covers them
  {
    const int nq = (a.ng + 1) >> 1;
    for (int q = wave; q < nq; q += 8) {
      const int c = 64 * q + lane;
      const int half = 16 * a.ng;  // chunks per 128 rows
      const int row0 = MODE == kModeGateUp ? (c < half ? 128 * nt : a.I + 128 * nt) : kPbBN * nt;
      const int cc = MODE == kModeGateUp && c >= half ? c - half : c;
      lds_dma16_buf(ssrc, row0 * a.ng * 2 + 16 * cc, reinterpret_cast<u32x4_t*>(sbuf) + 64 * q);
    }
  }
  // prologue: k tiles 0 .. kPbRing - 2 in flight, tile 0 landed
#pragma unroll
  for (int t = 0; t < kPbRing - 1; ++t) issue(t, t);
  wait_next();
  land(0, 0);
  lds_barrier();
  const int nkt_r = (nkt + kPbRing - 1) / kPbRing * kPbRing;
  for (int t0 = 0; t0 < nkt_r; t0 += kPbRing) {
#pragma unroll
    for (int r = 0; r < kPbRing; ++r) {
      const int t = t0 + r;
      // refill the slot k tile t - 1 used with tile t + kPbRing - 1 (inside
      // the multiplication when this wavefront has any)
      if (work && t < nkt)
        compute(t, r, t + kPbRing - 1, (r + kPbRing - 1) % kPbRing);
      else
        issue(t + kPbRing - 1, (r + kPbRing - 1) % kPbRing);
      wait_next();
      land(t + 1, (r + 1) % kPbRing);
      lds_barrier();
    }
  }
  // the tiles loaded past the end land before the epilogue reuses LDS; the
  // next item's index (fetched at the start of this one) is published by
  // the same barrier
  __builtin_amdgcn_s_waitcnt(vm_wait(0));
  if (tid == 0) *next_slot = next;
  lds_barrier();

  // epilogue: bf16 results -> wavefront-private LDS rows -> 16-byte stores
  if (MODE == kModeGateUp) {
    // 8 NF intermediate columns per wavefront (NF / 2 gate blocks and their
    // up blocks), bias order inside each 8-block
    constexpr int PITCH = 40;
    constexpr int H2 = NF / 2;
    uint16_t* ob = reinterpret_cast<uint16_t*>(smem) + wave * 64 * PITCH;
    float* red = reinterpret_cast<float*>(smem + 8 * 64 * PITCH * 2);  // [4][128]
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 16 * i + 4 * kb + q;
#pragma unroll
        for (int f = 0; f < H2; ++f) {
          const float gate = round_bf16(acc[i][f][q]);
          const float act = round_bf16(gelu_tanh_f32(gate));
          const float h = act * round_bf16(acc[i][f + H2][q]);
          const int c = 16 * f + j;
          ob[r * PITCH + (c & ~7) + bias_pos(c & 7)] = f32_to_bf16_bits(h);
        }
      }
    }
    // the wavefront reads back only what it wrote: no barrier needed.  Row
    // r's NF 16-byte chunks are held by NF consecutive lanes.
#pragma unroll
    for (int c4 = 0; c4 < MI * NF / 4; ++c4) {
      const int idx = lane + 64 * c4;
      const int r = idx / NF, cc = idx % NF;
      const int row = wm * RW + r;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ob + r * PITCH + 8 * cc);
      // intermediate column 128 nt + 8 NF wn + 8 cc + e: chunk
      // ch = NF wn + cc of tile nt, stored transposed at 4 (ch % 4) + ch / 4
      const int ch = NF * wn + cc;
      if (cols_ok && row < nrows)
        st16(a.out + (int64_t)(seg0 + row) * a.ldo + 128 * nt + 8 * (4 * (ch & 3) + (ch >> 2)), v);
      // the row's sum over this wavefront's columns (the values stored)
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
      float ps = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) ps += bf16_bits_to_f32(w4[q] & 0xFFFFu) + bf16_bits_to_f32(w4[q] >> 16);
      ps += __uint_as_float(__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(ps), 0xB1, 0xF, 0xF, false));
      if (NF == 4)
        ps += __uint_as_float(__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(ps), 0x4E, 0xF, 0xF, false));
      if (cc == 0) red[wn * kPbBM + row] = cols_ok ? ps : 0.f;
    }
    lds_barrier();
    if (tid < kPbBM && tid < nrows)
      a.cr_out[(int64_t)nt * a.ldc + seg0 + tid] =
          -136.0f * (((red[tid] + red[kPbBM + tid]) + red[2 * kPbBM + tid]) + red[3 * kPbBM + tid]);
  } else {
    // 16 NF output columns per wavefront
    constexpr int PITCH = 72;
    uint16_t* ob = reinterpret_cast<uint16_t*>(smem) + wave * 64 * PITCH;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int f = 0; f < NF; ++f)
          ob[(16 * i + 4 * kb + q) * PITCH + 16 * f + j] = f32_to_bf16_bits(acc[i][f][q]);
#pragma unroll
    for (int c8 = 0; c8 < MI * NF / 2; ++c8) {
      const int idx = lane + 64 * c8;
      const int r = idx / (2 * NF), cc = idx % (2 * NF);
      const int row = wm * RW + r;
      if (cols_ok && row < nrows) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ob + r * PITCH + 8 * cc);
        const int64_t orow = a.sorted_pos[seg0 + row];
        st16(a.out + orow * a.N + kPbBN * nt + 16 * NF * wn + 8 * cc, v);
      }
    }
  }
}

// Persistent grid of one workgroup per CU.  Items are (m-tile, n-tile) in
// m-tile-major order; XCD x (workgroups are dealt to the 8 XCDs in turn)
// owns a contiguous eighth of them.  Its P workgroups start on the run's
// first P items and then take the next one from the XCD's queue counter, so
// items of different cost (full, 64-row tails, half-width n-tiles) spread
// over the workgroups as they finish.  The queues start at zero
// (k_prefill_prep zeroes them before each gate_up; the last workgroup of
// each launch to leave resets its kernel's queues).
template <int MODE>
__global__ __launch_bounds__(kPbThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_prefill_bias(PrefillArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_item[2];
  const int tid = threadIdx.x;
  const int ntiles = ld_uniform(a.counters, 1);
  const int total = ntiles * a.n_nt;
  const int xcd = blockIdx.x & 7;
  const int chunk = (total + 7) >> 3;
  const int it_beg = xcd * chunk;
  const int it_end = min(total, it_beg + chunk);
  const int per_xcd = gridDim.x >> 3;
  const int q_beg = it_beg + per_xcd;  // the first item the queue hands out
  int* queue = a.queues + xcd;
  int* done = a.queues + 8;
  int slot = 0;
  int item = it_beg + (blockIdx.x >> 3);
  // (an index below the XCD's range could only come from a queue that was
  // not zeroed: stop rather than read outside the tile list)
  while (item >= it_beg && item < it_end) {
    const int next =
        tid == 0 ? q_beg + __hip_atomic_fetch_add(queue, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    const int mt = item / a.n_nt;
    const int nt = item - mt * a.n_nt;
    const int tile = ld_uniform(a.tiles, mt);
    const int e = tile >> 16;
    const int seg0 = ld_uniform(a.offsets, e) + (tile & 0xFFFF) * kPbBM;
    const int nrows = min(kPbBM, ld_uniform(a.offsets, e + 1) - seg0);
    const bool half_m = nrows <= 64;
    const bool half_n = MODE == kModeGateUp ? a.I - 128 * nt <= 64 : a.N - kPbBN * nt <= 128;
    int* nslot = &s_item[slot ^ 1];
    if (half_m) {
      if (half_n)
        pb_item<MODE, 2, 2>(a, smem, nt, e, seg0, nrows, nslot, next);
      else
        pb_item<MODE, 2, 4>(a, smem, nt, e, seg0, nrows, nslot, next);
    } else {
      if (half_n)
        pb_item<MODE, 4, 2>(a, smem, nt, e, seg0, nrows, nslot, next);
      else
        pb_item<MODE, 4, 4>(a, smem, nt, e, seg0, nrows, nslot, next);
    }
    slot ^= 1;
    item = __builtin_amdgcn_readfirstlane(s_item[slot]);
  }
  // the last workgroup to leave resets the queues for the next launch.  Every
  // other workgroup has taken its final index before counting itself out:
  // its loop ended on the value that fetch returned, so the fetch was
  // performed before the count was issued (relaxed order suffices; a
  // release here would write back the L2 of each workgroup's XCD)
  if (tid == 0) {
    const int d = __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == (int)gridDim.x - 1) {
#pragma unroll
      for (int x = 0; x < 9; ++x) __hip_atomic_store(a.queues + x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// persistent grid: the workgroups that fit on the device at once (a multiple
// of the 8 XCDs), at most one per item
int prefill_grid_size(const void* kern, int threads, size_t lds, int max_items) {
  int dev = 0, cus = 256, per_cu = 1;
  hipDeviceProp_t p;
  if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess &&
      p.multiProcessorCount > 0)
    cus = p.multiProcessorCount;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, lds) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  int g = cus * per_cu;
  if (max_items < g) g = max_items;
  return ((g + 7) / 8) * 8;
}

size_t prefill_bias_lds_bytes() {
  return (size_t)kPbRing * (kPbAStage + kPbBStage) * 16 + (size_t)(kPbRing + 1) * kPbBM * 4 +
         (size_t)kPbBN * kPbMaxNg * 2;
}

bool prefill_bias_supported(int ng) { return ng % 2 == 0 && ng <= kPbMaxNg; }

hipError_t launch_prefill_bias(int mode, PrefillArgs a, int max_mtiles, hipStream_t s) {
  if (max_mtiles <= 0) return hipSuccess;
  const size_t lds = prefill_bias_lds_bytes();
  if (mode == kModeGateUp) {
    auto kern = k_prefill_bias<kModeGateUp>;
    hipLaunchKernelGGL(kern, dim3(prefill_grid_size(reinterpret_cast<const void*>(kern), kPbThreads, lds,
                                                    max_mtiles * a.n_nt)),
                       dim3(kPbThreads), lds, s, a);
  } else {
    auto kern = k_prefill_bias<kModeDown>;
    hipLaunchKernelGGL(kern, dim3(prefill_grid_size(reinterpret_cast<const void*>(kern), kPbThreads, lds,
                                                    max_mtiles * a.n_nt)),
                       dim3(kPbThreads), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace w4a16
