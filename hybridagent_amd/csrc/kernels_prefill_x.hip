// Prefill-shaped W4A16 MoE expert GEMMs, exact form, for group sizes that are
// powers of two >= 32 (the released checkpoints' 32 and the benchmark's 128):
//
//   MODE = gateup : inter[s] = gelu(x[tok(s)] Wg^T) * (x[tok(s)] Wu^T)
//                   (quantization.py:112-120), rows s in expert-segment order
//   MODE = down   : dn[sorted_pos[s]] = inter[s] W_d^T   (quantization.py:122-127)
//
// Work item = (m-tile of up to 256 rows of one expert's segment, n-tile of
// 256 weight rows; gate_up: 128 gate rows + the matching 128 up rows).  A
// persistent grid of one 512-thread workgroup per CU: XCD x (workgroups are
// dealt to the 8 XCDs in turn) owns m-tiles x, x + 8, ... of the tile list
// (which lists the large tiles first) with all their n-tiles, and its
// workgroups take its items in turn.  Each of the eight wavefronts owns 32
// weight rows (gate_up: 16 gate + their 16 up rows) for all the item's
// rows: MB m-blocks of v_mfma_f32_32x32x16_bf16 accumulators (MB = 8 for
// 256 rows; 4, 2, 1 for segment tails of up to 128, 64, 32 rows).
//
// Per 64-wide k stage, all by direct global -> LDS loads of 16 bytes per
// lane (one instruction fills 1 KiB).  Every load of the main loop is one,
// all of one size, so they complete in the order they were issued and a
// partial vmcnt wait proves a stage landed (direct loads of 4 bytes were
// seen to finish ahead of 16-byte ones issued before them):
//   A  the item's activation rows, 8 rows x 128 bytes per instruction, rows
//      128 bytes apart with the 16-byte chunks XOR-swizzled by (row / 2) % 8
//      so that the fragment reads of 16 consecutive rows cover all LDS banks
//      once;
//   B  the packed words of the 256 weight rows (32 bytes each) and, per
//      row, the aligned 16 bytes of its scales that hold this stage's
//      group(s) (an aligned pair of bf16).
// A ring of three stages keeps two in flight while one is multiplied, and
// runs on across items: a workgroup's next item's first two stages load
// during the current item's last two, and its epilogue runs while they
// land.  Each
// lane dequantises the four packed words of its weight row that its four
// MFMA steps need exactly as the reference does -- bf16_RNE(q * s),
// q = u - 8 -- in registers; one B fragment feeds the MB MFMAs of its step.
// The lane layout of an MFMA step: lane l holds row (col) l % 32 and the
// 8 k of chunk 4 (l / 32) + s of the stage, for A and B alike.
//
// Epilogue: accumulators -> bf16 -> wavefront-private LDS rows (a region of
// their own, apart from the ring) -> 16-byte stores; gate_up pairs each gate
// column with its up column there and applies gelu_tanh(gate) * up with the
// reference's bf16 rounding points.
//
// While direct LDS loads are in flight the kernel issues no other vector
// memory load: row indices (gate_up: the next item's gathered token rows;
// down: the current item's output rows) come into an LDS table by a direct
// load of their own, one per stage (unused ones land in the junk block).
// (A direct LDS load and an ordinary load issued after it need not
// complete in that order, so a vmcnt wait counted for one could pass while
// the other is outstanding.)
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kPxWaves = 8;
constexpr int kPxThreads = 64 * kPxWaves;
constexpr int kPxBM = kPrefillXBM;           // 256 rows
constexpr int kPxBN = 32 * kPxWaves;         // 256 weight rows per item
constexpr int kPxKT = 64;                    // k per stage
constexpr int kPxStages = 3;
// LDS: the ring of stages, each A [256 rows][128 B] | B words [256 tile
// rows][32 B] | scale chunks [256 tile rows][16 B]; then 1 KiB that unused
// loads land in; the row-index table (512 ints from a 16-byte-aligned
// start: sorted_pos[s & ~3 ..] for a segment starting at s); the epilogue
// rows, 32 rows x 32 bf16 per wavefront
constexpr int kPxBOff = kPxBM * kPxKT * 2;
constexpr int kPxSOff = kPxBOff + kPxBN * kPxKT / 2;
constexpr int kPxStageBytes = kPxSOff + kPxBN * 16;
constexpr int kPxJunk = kPxStages * kPxStageBytes;
constexpr int kPxTable = kPxJunk + 1024;  // 512 row indices
constexpr int kPxEpiOff = kPxTable + 2048;
constexpr int kPxEpiBytes = 32 * 64;
constexpr int kPxLds = kPxEpiOff + kPxWaves * kPxEpiBytes;
// direct A loads per wavefront and stage (tiles of fewer rows send the
// unused ones to the junk block, so every stage counts the same loads),
// then one B-word, one scale-pair and one row-index load
constexpr int kPxNA = 4;
constexpr int kPxLoads = kPxNA + 3;

// s_waitcnt immediate for vmcnt <= n with expcnt and lgkmcnt not waited for
// (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int px_vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Workgroup barrier for LDS data only: each wavefront waits for its own LDS
// operations, then meets the others.  (__syncthreads() would also wait for
// every global load in flight, the direct LDS loads of the next stages
// included.)
__device__ __forceinline__ void px_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// direct global -> LDS load: lane l's 16 bytes land at lds_dst + 16 l
__device__ __forceinline__ void px_dma16(__amdgpu_buffer_rsrc_t rsrc, int voff, int soff, void* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds_dst, 16,
                                          voff, soff, 0, 0);
}

// byte b of v as a float (v_cvt_f32_ubyte<b>; written out because the
// compiler otherwise extracts bytes 1..3 with a separate v_bfe_u32 first)
template <int B>
__device__ __forceinline__ float cvt_ubyte(uint32_t v) {
  float r;
  if (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  if (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  if (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  if (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// Exact dequantisation of one packed word (k = 8 j .. 8 j + 7 of one weight
// row) into 8 bf16 in natural k order: bf16_RNE(q * s), q = u - 8, computed
// as fma(u, s, -8 s) -- both products are exact in fp32 (|u| <= 15, s has 8
// significant bits) -- then rounded by v_cvt_pk_bf16_f32.  m8 = -8 s.
__device__ __forceinline__ u32x4_t dequant_word(uint32_t w, float s, float m8) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
  u32x4_t r;
  r.x = pack_bf16x2(__builtin_fmaf(cvt_ubyte<0>(lo), s, m8), __builtin_fmaf(cvt_ubyte<0>(hi), s, m8));
  r.y = pack_bf16x2(__builtin_fmaf(cvt_ubyte<1>(lo), s, m8), __builtin_fmaf(cvt_ubyte<1>(hi), s, m8));
  r.z = pack_bf16x2(__builtin_fmaf(cvt_ubyte<2>(lo), s, m8), __builtin_fmaf(cvt_ubyte<2>(hi), s, m8));
  r.w = pack_bf16x2(__builtin_fmaf(cvt_ubyte<3>(lo), s, m8), __builtin_fmaf(cvt_ubyte<3>(hi), s, m8));
  return r;
}

__device__ __forceinline__ f32x16_t mfma32x(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

}  // namespace


// One work item: (m-tile, n-tile) and what that fixes.
struct PxItem {
  int nt, e, seg0, nrows, mb;
};

__device__ __forceinline__ PxItem px_item_info(const PrefillArgs& a, int xcd, int item) {
  PxItem it;
  const int lm = item / a.n_nt;
  it.nt = item - lm * a.n_nt;
  const int tile = ld_uniform(a.tiles, xcd + 8 * lm);
  it.e = tile >> 16;
  it.seg0 = ld_uniform(a.offsets, it.e) + (tile & 0xFFFF) * kPxBM;
  it.nrows = min(kPxBM, ld_uniform(a.offsets, it.e + 1) - it.seg0);
  it.mb = it.nrows > 128 ? 8 : it.nrows > 64 ? 4 : it.nrows > 32 ? 2 : 1;
  return it;
}

// A lane's load sources for one item (and the destinations, which are
// wavefront-uniform).
struct PxLoads {
  __amdgpu_buffer_rsrc_t wsrc, ssrc;
  int avoff[kPxNA], adst[kPxNA];
  int bvoff, svoff, sdst;
};

// weight row of tile row tr of n-tile nt (gate_up: wavefront w's tile rows
// 32 w .. 32 w + 31 are gate rows 128 nt + 16 w .. + 15, then the matching
// up rows; rows past the matrix repeat its last row, their results are
// dropped)
template <int MODE>
__device__ __forceinline__ int px_weight_row(const PrefillArgs& a, int nt, int tr) {
  if (MODE == kModeGateUp) {
    const int w = tr >> 5, cc = tr & 31;
    const int col = min(128 * nt + 16 * w + (cc & 15), a.I - 1);
    return cc < 16 ? col : a.I + col;
  }
  return min(kPxBN * nt + tr, a.N - 1);
}

// gate_up reads the item's gathered rows from the LDS table, which must
// hold this item's rows (row r at entry seg0 % 4 + r)
template <int MODE>
__device__ __forceinline__ PxLoads px_loads(const PrefillArgs& a, const PxItem& it, const unsigned char* smem) {
  PxLoads L;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // A: instruction j = wave + 8 i brings rows 8 j .. 8 j + 7; lane l takes
  // row 8 j + l / 8 into LDS slot l % 8, i.e. chunk (l % 8) ^ ((row / 2) % 8)
  // of the row (rows past the segment repeat its last row).
  const int* table = reinterpret_cast<const int*>(smem + kPxTable);
#pragma unroll
  for (int i = 0; i < kPxNA; ++i) {
    const int j = wave + 8 * i;
    const bool real = j < 4 * it.mb;
    const int r = 8 * j + (lane >> 3);
    const int rr = min(r, it.nrows - 1);
    const int64_t src = MODE == kModeGateUp ? (real ? table[(it.seg0 & 3) + rr] : 0) / a.topk : it.seg0 + rr;
    const int chunk = (lane & 7) ^ ((r >> 1) & 7);
    L.avoff[i] = real ? (int)(src * a.lda * 2) + 16 * chunk : 0;
    L.adst[i] = real ? j * 1024 : kPxJunk;
  }
  // B words: instruction `wave` brings tile rows 32 wave .. + 31, lane l row
  // 32 wave + l / 2, bytes 16 (l % 2) of the stage's 32
  const int K2 = a.K >> 1;  // packed bytes per weight row
  L.wsrc = make_rsrc(reinterpret_cast<const uint32_t*>(a.wp) + (int64_t)it.e * a.N * (a.K >> 3),
                     (uint32_t)a.N * K2);
  L.bvoff = px_weight_row<MODE>(a, it.nt, 32 * wave + (lane >> 1)) * K2 + 16 * (lane & 1);
  // scale chunks: waves 0..3 bring tile rows 64 wave + l, the aligned 16
  // bytes holding the stage's scale pair (the stage adds 2 x the pair's
  // group index, the lane rounds down to 16 bytes); waves 4..7 load one
  // unused block.  The descriptor starts at the expert's scales rounded
  // down to 16 bytes; svoff carries the difference.
  const uintptr_t sbase = reinterpret_cast<uintptr_t>(a.ws + (int64_t)it.e * a.N * a.ng);
  L.ssrc = make_rsrc(reinterpret_cast<const void*>(sbase & ~uintptr_t(15)), (uint32_t)a.N * a.ng * 2u + 16u);
  const bool sreal = wave < 4;
  L.svoff = sreal ? (int)(sbase & 15) + px_weight_row<MODE>(a, it.nt, 64 * wave + lane) * a.ng * 2 : 0;
  L.sdst = sreal ? kPxSOff + 1024 * wave : kPxJunk;
  return L;
}

// The kPxLoads direct loads of stage kt of an item into ring slot `slot`;
// with tseg >= 0 the last ones of wavefronts 0 and 1 bring the row indices
// sorted_pos[tseg & ~3 ..] (512 entries; past the routed rows they read as
// zero, readers clamp to the segment) into the LDS table, otherwise they
// land in the junk block.
__device__ __forceinline__ void px_issue(const PrefillArgs& a, const PxLoads& L, unsigned char* smem, int kt,
                                         int slot, int tseg) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned char* st = smem + slot * kPxStageBytes;
#pragma unroll
  for (int i = 0; i < kPxNA; ++i)
    px_dma16(make_rsrc(a.act, (uint32_t)a.act_bytes), L.avoff[i], kt * (kPxKT * 2),
             L.adst[i] == kPxJunk ? smem + kPxJunk : st + L.adst[i]);
  px_dma16(L.wsrc, L.bvoff, kt * (kPxKT / 2), st + kPxBOff + wave * 1024);
  const int gpair = ((kt * kPxKT) >> a.gshift) & ~1;
  px_dma16(L.ssrc, (L.svoff + 2 * gpair) & ~15, 0, L.sdst == kPxJunk ? smem + kPxJunk : st + L.sdst);
  {
    const bool treal = tseg >= 0 && wave < 2;
    const __amdgpu_buffer_rsrc_t tsrc = make_rsrc(a.sorted_pos, (uint32_t)a.rows_total * 4u);
    px_dma16(tsrc, treal ? 4 * ((tseg & ~3) + 256 * wave + 4 * lane) : 0, 0,
             treal ? smem + kPxTable + 1024 * wave : smem + kPxJunk);
  }
}

// Multiply one item.  On entry its stages 0 and 1 are issued into slots p0
// and p0 + 1; with `first` stage 0 has not been waited for.  Its last two
// iterations (peeled, so the next item's load sources are live only there)
// issue the next item's stages 0 and 1 (or, when there is none, its own
// last stage again, unused), so on return those are in flight.
template <int MODE, int MB>
__device__ __forceinline__ void px_run(const PrefillArgs& a, unsigned char* smem, const PxItem& it,
                                       const PxItem& nx, bool has_next, int p0, bool first) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nkt = a.K / kPxKT;
  const int h = lane >> 5;  // which half of the step's 16 k this lane holds
  const int c = lane & 31;  // row (A) / column (B) inside a 32-block
  const int gshift = a.gshift;
  const int nt = it.nt, seg0 = it.seg0, nrows = it.nrows;

  // this lane's reads: A fragment of block mb, step s -> row 32 mb + c,
  // chunk 4 h + s at slot chunk ^ ((c / 2) % 8); B words and scale pair of
  // tile row 32 wave + c
  int aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = c * 128 + 16 * ((4 * h + s) ^ ((c >> 1) & 7));
  const int boff = kPxBOff + (32 * wave + c) * 32 + 16 * h;
  // the scale chunk of tile row 32 wave + c; the pair sits at byte
  // (2 (row ng + pair group)) % 16 of it
  const int soff = kPxSOff + (32 * wave + c) * 16;
  const int srow2 = (int)(reinterpret_cast<uintptr_t>(a.ws + (int64_t)it.e * a.N * a.ng) & 15) +
                    px_weight_row<MODE>(a, nt, 32 * wave + c) * a.ng * 2;
  auto soff_of = [&](int t) -> int { return soff + ((srow2 + 2 * (((t * kPxKT) >> gshift) & ~1)) & 15); };
  // wavefronts whose columns lie past the matrix (gate_up's last n-tile
  // when I % 128 == 64) do no MFMA work and store nothing
  const bool work = MODE == kModeGateUp ? 128 * nt + 16 * wave < a.I : kPxBN * nt + 32 * wave < a.N;

  f32x16_t acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[i][q] = 0.f;

  auto scale_of = [&](int t, uint32_t sp) -> float {
    const int g = (t * kPxKT + 32 * h) >> gshift;
    const int sel = g - (((t * kPxKT) >> gshift) & ~1);  // 0 or 1
    return bf16_bits_to_f32((sp >> (16 * sel)) & 0xFFFFu);
  };
  auto read_a = [&](const unsigned char* st, int s, u32x4_t* af) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) af[mb] = *reinterpret_cast<const u32x4_t*>(st + mb * 4096 + aoff[s]);
  };
  auto mfmas = [&](const u32x4_t* af, u32x4_t bf) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma32x(af[mb], bf, acc[mb]);
  };
  auto stage_ptr = [&](int sl) -> const unsigned char* { return smem + sl * kPxStageBytes; };
  auto wait_and_sync = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(px_vm_wait(kPxLoads));
    __builtin_amdgcn_sched_barrier(0);
    px_barrier();
  };

  if (first) wait_and_sync();  // stage 0 landed (stage 1 may still be loading)
  // Software pipeline: each A fragment register is reloaded with the next
  // step's fragment right after the MFMA that reads it, and the next step's
  // B fragment is dequantised while the current step's MFMAs run.  Stage
  // t's last-step fragments are in registers before the barrier that ends
  // the stage, so after it each MFMA of that step is followed by the read
  // of stage t + 1's first fragment for the same block.
  u32x4_t af[MB];
  u32x4_t bw = {0u, 0u, 0u, 0u};
  float sc = 0.f;
  if (work) {
    read_a(stage_ptr(p0), 0, af);
    bw = *reinterpret_cast<const u32x4_t*>(stage_ptr(p0) + boff);
    sc = scale_of(0, *reinterpret_cast<const uint32_t*>(stage_ptr(p0) + soff_of(0)));
  }
  int slot = p0;
  int slot2 = p0 + 2 >= kPxStages ? p0 + 2 - kPxStages : p0 + 2;
  // one k stage: refill the slot stage t - 1 used (issue(slot2)), multiply
  // stage t, wait for stage t + 1 and meet the other wavefronts
  auto iter = [&](int t, auto issue) {
    issue(slot2);
    const int nslot = slot == kPxStages - 1 ? 0 : slot + 1;
    if (work) {
      const unsigned char* st = stage_ptr(slot);
      const float m8 = -8.0f * sc;
      const uint32_t wv[4] = {bw.x, bw.y, bw.z, bw.w};
      u32x4_t bf = dequant_word(wv[0], sc, m8);
#pragma unroll
      for (int s2 = 0; s2 < 3; ++s2) {
        const u32x4_t bfn = dequant_word(wv[s2 + 1], sc, m8);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          acc[mb] = mfma32x(af[mb], bf, acc[mb]);
          af[mb] = *reinterpret_cast<const u32x4_t*>(st + mb * 4096 + aoff[s2 + 1]);
        }
        bf = bfn;
      }
      wait_and_sync();  // stage t + 1 landed (stage t + 2 may still be loading)
      if (t + 1 < nkt) {
        const unsigned char* sn = stage_ptr(nslot);
        bw = *reinterpret_cast<const u32x4_t*>(sn + boff);
        const uint32_t sp = *reinterpret_cast<const uint32_t*>(sn + soff_of(t + 1));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          acc[mb] = mfma32x(af[mb], bf, acc[mb]);
          af[mb] = *reinterpret_cast<const u32x4_t*>(sn + mb * 4096 + aoff[0]);
        }
        sc = scale_of(t + 1, sp);
      } else {
        mfmas(af, bf);
      }
    } else {
      wait_and_sync();
    }
    slot = nslot;
    slot2 = slot2 == kPxStages - 1 ? 0 : slot2 + 1;
  };
  // the row-index table: gate_up loads the next item's rows with stage
  // nkt - 2 (issued in iteration nkt - 4, landed before iteration nkt - 2
  // builds the next item's load sources); down loads its own output rows with
  // stage 3 (iteration 1: every wavefront is past the previous epilogue)
  auto table_seg = [&](int t) -> int {
    if (MODE == kModeGateUp) return (t == nkt - 4 && has_next) ? nx.seg0 : -1;
    return t == 1 ? seg0 : -1;
  };
  {
    const PxLoads lc = px_loads<MODE>(a, it, smem);
    for (int t = 0; t + 2 < nkt; ++t) iter(t, [&](int sl) { px_issue(a, lc, smem, t + 2, sl, table_seg(t)); });
    if (!has_next) {
      iter(nkt - 2, [&](int sl) { px_issue(a, lc, smem, nkt - 1, sl, -1); });
      iter(nkt - 1, [&](int sl) { px_issue(a, lc, smem, nkt - 1, sl, -1); });
    }
  }
  if (has_next) {
    const PxLoads ln = px_loads<MODE>(a, nx, smem);
    iter(nkt - 2, [&](int sl) { px_issue(a, ln, smem, 0, sl, -1); });
    iter(nkt - 1, [&](int sl) { px_issue(a, ln, smem, 1, sl, -1); });
  }
  if (!work) return;

  // ---- epilogue, in passes of 32 rows (one m-block).  Lane l holds
  // column c of block mb at rows 32 mb + 8 (q / 4) + 4 h + q % 4
  // (q = 0..15).  Each wavefront writes its rows x 32 columns as bf16 into
  // its own 64-byte LDS rows, then reads 16 bytes per lane back for the
  // global stores (it reads only what it wrote: no barrier).  The region is
  // not part of the ring, so the next item's stages land meanwhile.
  constexpr int HB = 1;  // m-blocks per pass
  constexpr int PR = 32 * HB;          // rows per pass
  uint16_t* ob = reinterpret_cast<uint16_t*>(smem + kPxEpiOff + wave * kPxEpiBytes);
#pragma unroll
  for (int p = 0; p < MB / HB; ++p) {
#pragma unroll
    for (int mb = 0; mb < HB; ++mb)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int row = 32 * mb + 8 * (q >> 2) + 4 * h + (q & 3);
        ob[row * 32 + c] = f32_to_bf16_bits(acc[p * HB + mb][q]);
      }
    if (MODE == kModeGateUp) {
      // row r, half hp: gate columns 8 hp .. 8 hp + 7 (bytes 16 hp) and
      // their up columns (bytes 32 + 16 hp) -> 8 intermediate values
#pragma unroll
      for (int itr = 0; itr < PR * 2 / 64; ++itr) {
        const int idx = lane + 64 * itr;
        const int row = idx >> 1, hp = idx & 1;
        const u32x4_t gv = *reinterpret_cast<const u32x4_t*>(ob + row * 32 + 8 * hp);
        const u32x4_t uv = *reinterpret_cast<const u32x4_t*>(ob + row * 32 + 16 + 8 * hp);
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
        uint32_t hw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g0 = bf16_bits_to_f32(gw[q] & 0xFFFFu), g1 = bf16_bits_to_f32(gw[q] >> 16);
          const float u0 = bf16_bits_to_f32(uw[q] & 0xFFFFu), u1 = bf16_bits_to_f32(uw[q] >> 16);
          hw[q] = pack_bf16x2(round_bf16(gelu_tanh_f32(g0)) * u0, round_bf16(gelu_tanh_f32(g1)) * u1);
        }
        const int grow = PR * p + row;
        if (grow < nrows)
          st16(a.out + (int64_t)(seg0 + grow) * a.ldo + 128 * nt + 16 * wave + 8 * hp,
               u32x4_t{hw[0], hw[1], hw[2], hw[3]});
      }
    } else {
      // output rows: dn row sorted_pos[seg0 + row], from the LDS table
      const int* table = reinterpret_cast<const int*>(smem + kPxTable);
#pragma unroll
      for (int itr = 0; itr < PR * 4 / 64; ++itr) {
        const int idx = lane + 64 * itr;
        const int row = idx >> 2, q4 = idx & 3;
        const int grow = PR * p + row;
        if (grow < nrows) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ob + row * 32 + 8 * q4);
          st16(a.out + (int64_t)table[(seg0 & 3) + grow] * a.N + kPxBN * nt + 32 * wave + 8 * q4, v);
        }
      }
    }
  }
}

template <int MODE>
__device__ __forceinline__ void px_dispatch(const PrefillArgs& a, unsigned char* smem, const PxItem& it,
                                            const PxItem& nx, bool has_next, int p0, bool first) {
  if (it.mb == 8)
    px_run<MODE, 8>(a, smem, it, nx, has_next, p0, first);
  else if (it.mb == 4)
    px_run<MODE, 4>(a, smem, it, nx, has_next, p0, first);
  else if (it.mb == 2)
    px_run<MODE, 2>(a, smem, it, nx, has_next, p0, first);
  else
    px_run<MODE, 1>(a, smem, it, nx, has_next, p0, first);
}

// Persistent grid, one workgroup per CU; workgroup b of XCD x = b % 8 takes
// that XCD's local items b / 8, b / 8 + P, b / 8 + 2 P, ... (P = workgroups
// per XCD).  Local item i is n-tile i % n_nt of the XCD's m-tile i / n_nt,
// global m-tile x + 8 (i / n_nt): the large items come first, the small ones
// fill in at the end, and the items of an m-tile run side by side on the
// XCD's workgroups.
template <int MODE>
__global__ __launch_bounds__(kPxThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_prefill_x(PrefillArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int ntiles = ld_uniform(a.counters, 1);
  const int xcd = blockIdx.x & 7;
  const int n_local = ntiles > xcd ? (ntiles - xcd + 7) >> 3 : 0;  // this XCD's m-tiles
  const int it_end = n_local * a.n_nt;
  const int step = gridDim.x >> 3;
  int item = blockIdx.x >> 3;
  if (item >= it_end) return;
  const int nkt = a.K / kPxKT;
  PxItem cur = px_item_info(a, xcd, item);
  if (MODE == kModeGateUp) {
    // the first item's gathered rows into the table (nothing else in flight)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t tsrc = make_rsrc(a.sorted_pos, (uint32_t)a.rows_total * 4u);
    if (wave < 2) px_dma16(tsrc, 4 * ((cur.seg0 & ~3) + 256 * wave + 4 * lane), 0, smem + kPxTable + 1024 * wave);
    __builtin_amdgcn_s_waitcnt(px_vm_wait(0));
    px_barrier();
  }
  {
    const PxLoads lc = px_loads<MODE>(a, cur, smem);
    px_issue(a, lc, smem, 0, 0, -1);
    px_issue(a, lc, smem, 1, 1, -1);
  }
  int p0 = 0;
  bool first = true;
  for (;;) {
    const int nitem = item + step;
    const bool has_next = nitem < it_end;
    const PxItem nxt = has_next ? px_item_info(a, xcd, nitem) : cur;
    px_dispatch<MODE>(a, smem, cur, nxt, has_next, p0, first);
    if (!has_next) break;
    item = nitem;
    cur = nxt;
    p0 = (p0 + nkt) % kPxStages;
    first = false;
  }
  // the loads issued past the last stage land before the workgroup leaves
  __builtin_amdgcn_s_waitcnt(px_vm_wait(0));
}

size_t prefill_x_lds_bytes() { return (size_t)kPxLds; }

// H and I multiples of the 64-wide stage, at least four stages; G a power of two >= 32 whose
// group counts per row are even for both matrices (a stage's scale pair is
// one aligned dword)
bool prefill_x_supported(int64_t H, int64_t I, int64_t G) {
  if (H % kPxKT != 0 || I % kPxKT != 0 || H < 4 * kPxKT || I < 4 * kPxKT || G < 32 || (G & (G - 1)) != 0)
    return false;
  const int64_t ng_h = (H + G - 1) / G, ng_i = (I + G - 1) / G;
  return ng_h % 2 == 0 && ng_i % 2 == 0;
}

hipError_t launch_prefill_x(int mode, PrefillArgs a, int max_mtiles, hipStream_t s) {
  if (max_mtiles <= 0) return hipSuccess;
  const size_t lds = prefill_x_lds_bytes();
  if (mode == kModeGateUp) {
    auto kern = k_prefill_x<kModeGateUp>;
    hipLaunchKernelGGL(kern, dim3(prefill_grid_size(reinterpret_cast<const void*>(kern), kPxThreads, lds,
                                                    max_mtiles * a.n_nt)),
                       dim3(kPxThreads), lds, s, a);
  } else {
    auto kern = k_prefill_x<kModeDown>;
    hipLaunchKernelGGL(kern, dim3(prefill_grid_size(reinterpret_cast<const void*>(kern), kPxThreads, lds,
                                                    max_mtiles * a.n_nt)),
                       dim3(kPxThreads), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace w4a16
