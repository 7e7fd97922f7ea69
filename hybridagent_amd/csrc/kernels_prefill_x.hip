// Prefill-shaped W4A16 MoE expert GEMMs, exact form, for group sizes that are
// powers of two >= 32 (the released checkpoints' 32 and the benchmark's 128):
//
//   MODE = gateup : inter[s] = gelu(x[tok(s)] Wg^T) * (x[tok(s)] Wu^T)
//                   (quantization.py:112-120), rows s in expert-segment order
//   MODE = down   : dn[sorted_pos[s]] = inter[s] W_d^T   (quantization.py:122-127)
//
// Work item = (m-tile of up to 256 rows of one expert's segment, n-tile of
// 256 weight rows; gate_up: 128 gate rows + the matching 128 up rows).  A
// persistent grid of one 512-thread workgroup per CU takes the items from a
// work queue (the tile list lists the large tiles first): for down, XCD x
// (workgroups are dealt to the 8 XCDs in turn) owns m-tiles x, x + 8, ...
// with all their n-tiles and a queue of its own; gate_up has one queue for
// the chip.  Each of the eight wavefronts owns 32
// weight rows (gate_up: 16 gate + their 16 up rows) for all the item's
// rows: MB m-blocks of v_mfma_f32_32x32x16_bf16 accumulators (MB = 8 for
// 256 rows; 4, 2, 1 for segment tails of up to 128, 64, 32 rows).  A tail of
// at most 32 rows (most of them are whole experts of few rows) is a wide
// item of three n-tiles: its stages carry three n-tiles' weights, so the
// per-stage cost that such an item pays for little MFMA work is paid once
// for three n-tiles, and each output is the one-n-tile item's bit for bit.
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
// runs on across items: a workgroup issues its next item's first two stages
// before the current item's epilogue, which runs while they land.  Each
// lane dequantises the four packed words of its weight row that its four
// MFMA steps need exactly as the reference does -- bf16_RNE(q * s),
// q = u - 8 -- in registers; one B fragment feeds the MB MFMAs of its step.
// The lane layout of an MFMA step: lane l holds row (col) l % 32 and the
// 8 k of chunk 4 (l / 32) + s of the stage, for A and B alike.
//
// The MFMAs compute D[weight row][activation row] (dequantised weights as
// the A operand), so each lane ends with four consecutive output columns of
// one activation row per register quad: the epilogue stores 8 bytes per
// lane straight from registers; gate_up finds each gate column's up column
// in the same lane and applies gelu_tanh(gate) * up with the reference's
// bf16 rounding points.
//
// While direct LDS loads are in flight the kernel issues no other vector
// memory load: row indices (gate_up: the next item's gathered token rows;
// down: the current item's output rows) come into an LDS table by a direct
// load of their own with the item's second-to-last stage.  (A direct LDS
// load and an ordinary load issued after it need not complete in that
// order, so a vmcnt wait counted for one could pass while the other is
// outstanding.)  Each wavefront issues only the loads it needs; a stage's
// wait counts the loads that wavefront issued after it.
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
// rows][32 B] | scale chunks [256 tile rows][16 B]; the row-index table
// (512 ints from a 16-byte-aligned start: sorted_pos[s & ~3 ..] for a
// segment starting at s); down's epilogue rows
constexpr int kPxBOff = kPxBM * kPxKT * 2;
constexpr int kPxSOff = kPxBOff + kPxBN * kPxKT / 2;
constexpr int kPxStageBytes = kPxSOff + kPxBN * 16;
constexpr int kPxTable = kPxStages * kPxStageBytes;  // 512 row indices
// down's epilogue rows: 32 rows x 32 bf16 per wavefront, rows 80 bytes
// apart (the 8-byte writes of 32 rows spread over the banks)
constexpr int kPxEpiOff = kPxTable + 2048;
constexpr int kPxEpiPitch = 80;
constexpr int kPxEpiBytes = 32 * kPxEpiPitch;
// the item index a workgroup takes from its XCD's queue (one int)
constexpr int kPxQSlot = kPxEpiOff + kPxWaves * kPxEpiBytes;
constexpr int kPxLds = kPxQSlot + 16;
// at most four direct A loads per wavefront and stage (fewer for tiles of
// fewer rows), then one B-word load and one scale-chunk load (wavefronts
// 0..3)
constexpr int kPxNA = 4;
// Wide items: a segment tail of at most kPrefillTinyRows rows (one m-block,
// listed last by the sort) takes kPxWide n-tiles at once, so its per-stage
// latency is paid once for three n-tiles' weights.  Its stage holds 32
// activation rows (4 KiB of the A region); the other n-tiles' words and
// scale chunks go in the rest of that region: n-tile b of the item has its
// words at px_wide_b(b) and its scale chunks at px_wide_s(b).
constexpr int kPxWide = 3;
constexpr int px_wide_b(int b) { return b == 0 ? kPxBOff : 4096 + 8192 * (b - 1); }
constexpr int px_wide_s(int b) { return b == 0 ? kPxSOff : 4096 + 8192 * (kPxWide - 1) + 4096 * (b - 1); }
static_assert(px_wide_s(kPxWide - 1) + 4096 <= kPxBOff, "a wide stage's blocks fit in the A region");
static_assert(kPrefillTinyRows == 32, "a wide item is one 32-row m-block");


// s_waitcnt immediate for vmcnt <= n with expcnt and lgkmcnt not waited for
// (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int px_vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// s_waitcnt vmcnt(n) for a wavefront-uniform n <= 7
__device__ __forceinline__ void px_wait_vm(int n) {
  switch (n) {
    case 1: __builtin_amdgcn_s_waitcnt(px_vm_wait(1)); break;
    case 2: __builtin_amdgcn_s_waitcnt(px_vm_wait(2)); break;
    case 3: __builtin_amdgcn_s_waitcnt(px_vm_wait(3)); break;
    case 4: __builtin_amdgcn_s_waitcnt(px_vm_wait(4)); break;
    case 5: __builtin_amdgcn_s_waitcnt(px_vm_wait(5)); break;
    case 6: __builtin_amdgcn_s_waitcnt(px_vm_wait(6)); break;
    case 7: __builtin_amdgcn_s_waitcnt(px_vm_wait(7)); break;
    default: __builtin_amdgcn_s_waitcnt(px_vm_wait(0)); break;
  }
}

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

__device__ __forceinline__ f32x16_t mfma32x(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

}  // namespace


// One work item: (m-tile, first n-tile, n-tiles nb) and what that fixes.
struct PxItem {
  int nt, e, seg0, nrows, mb, nb;
};

// Item `item` of a queue whose m-tiles are tile list entries x0, x0 + xs, ...:
// m-tiles [t0, t1) of the queue (the tails of at most kPrefillTinyRows rows)
// have n_wide items of kPxWide n-tiles each (n-tiles past the matrix compute
// on its last rows and store nothing), the others n_nt items of one n-tile.
__device__ __forceinline__ PxItem px_item_info(const PrefillArgs& a, int x0, int xs, int t0, int t1, int n_wide,
                                               int item) {
  PxItem it;
  const int i0 = t0 * a.n_nt, i1 = i0 + (t1 - t0) * n_wide;
  int lm;
  it.nb = 1;
  if (item < i0) {
    lm = item / a.n_nt;
    it.nt = item - lm * a.n_nt;
  } else if (item < i1) {
    const int j = item - i0;
    const int q = j / n_wide;
    lm = t0 + q;
    it.nt = kPxWide * (j - q * n_wide);
    it.nb = kPxWide;
  } else {
    const int j = item - i1;
    const int q = j / a.n_nt;
    lm = t1 + q;
    it.nt = j - q * a.n_nt;
  }
  const int tile = ld_uniform(a.tiles, x0 + xs * lm);
  it.e = tile >> 16;
  it.seg0 = ld_uniform(a.offsets, it.e) + (tile & 0xFFFF) * kPxBM;
  it.nrows = min(kPxBM, ld_uniform(a.offsets, it.e + 1) - it.seg0);
  it.mb = it.nrows > 128 ? 8 : it.nrows > 64 ? 4 : it.nrows > 32 ? 2 : 1;
  return it;
}

// A lane's load sources for one item; na = the wavefront's A loads per
// stage, n = all its loads per stage (both wavefront-uniform).
struct PxLoads {
  __amdgpu_buffer_rsrc_t wsrc, ssrc;
  int avoff[kPxNA];
  int bvoff, bstride, svoff;
  int na, n;
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
  L.na = 0;
#pragma unroll
  for (int i = 0; i < kPxNA; ++i) {
    const int j = wave + 8 * i;
    const bool real = j < 4 * it.mb;
    L.na += real ? 1 : 0;
    const int r = 8 * j + (lane >> 3);
    const int rr = min(r, it.nrows - 1);
    const int64_t src = MODE == kModeGateUp ? (real ? table[(it.seg0 & 3) + rr] : 0) / a.topk : it.seg0 + rr;
    const int chunk = (lane & 7) ^ ((r >> 1) & 7);
    L.avoff[i] = real ? (int)(src * a.lda * 2) + 16 * chunk : 0;
  }
  L.n = L.na + 1 + (wave < 4 ? 1 : 0);
  // B words: instruction `wave` brings tile rows 32 wave .. + 31, lane l row
  // 32 wave + l / 2, bytes 16 (l % 2) of the stage's 32
  const int K2 = a.K >> 1;  // packed bytes per weight row
  if (a.wt != nullptr) {
    // tiled copy: the item's stage kt is the 8 KiB block (nt, kt) of the
    // expert, tile rows in order, so instruction `wave` reads one KiB
    const int nkt = a.K / kPxKT;
    const int64_t per_e = (int64_t)a.n_nt * nkt * 2048;  // int32 words
    L.wsrc = make_rsrc(reinterpret_cast<const uint32_t*>(a.wt) + (int64_t)it.e * per_e, (uint32_t)(per_e * 4));
    L.bvoff = it.nt * nkt * 8192 + wave * 1024 + 16 * lane;
    L.bstride = 8192;
  } else {
    L.wsrc = make_rsrc(reinterpret_cast<const uint32_t*>(a.wp) + (int64_t)it.e * a.N * (a.K >> 3),
                       (uint32_t)a.N * K2);
    L.bvoff = px_weight_row<MODE>(a, it.nt, 32 * wave + (lane >> 1)) * K2 + 16 * (lane & 1);
    L.bstride = kPxKT / 2;
  }
  // scale chunks: waves 0..3 bring tile rows 64 wave + l, the aligned 16
  // bytes holding the stage's scale pair (the stage adds 2 x the pair's
  // group index, the lane rounds down to 16 bytes).  The descriptor starts
  // at the expert's scales rounded down to 16 bytes; svoff carries the
  // difference.
  const uintptr_t sbase = reinterpret_cast<uintptr_t>(a.ws + (int64_t)it.e * a.N * a.ng);
  L.ssrc = make_rsrc(reinterpret_cast<const void*>(sbase & ~uintptr_t(15)), (uint32_t)a.N * a.ng * 2u + 16u);
  const bool sreal = wave < 4;
  L.svoff = sreal ? (int)(sbase & 15) + px_weight_row<MODE>(a, it.nt, 64 * wave + lane) * a.ng * 2 : 0;
  return L;
}

// Part `part` (0..3, issued before MFMA step `part`) of the direct loads of
// stage kt of an item into ring slot `slot`, L.n loads in all: part p brings
// A load p (if this wavefront has one), part 0 also the B words, part 1 the
// scale chunks.
__device__ __forceinline__ void px_issue(const PrefillArgs& a, const PxLoads& L, unsigned char* smem, int kt,
                                         int slot, int part) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned char* st = smem + slot * kPxStageBytes;
  if (part < L.na)
    px_dma16(make_rsrc(a.act, (uint32_t)a.act_bytes), L.avoff[part], kt * (kPxKT * 2),
             st + (wave + 8 * part) * 1024);
  if (part == 0) px_dma16(L.wsrc, L.bvoff, kt * L.bstride, st + kPxBOff + wave * 1024);
  if (part == 1 && wave < 4) {
    const int gpair = ((kt * kPxKT) >> a.gshift) & ~1;
    px_dma16(L.ssrc, (L.svoff + 2 * gpair) & ~15, 0, st + kPxSOff + 1024 * wave);
  }
}

__device__ __forceinline__ void px_issue_all(const PrefillArgs& a, const PxLoads& L, unsigned char* smem, int kt,
                                             int slot) {
#pragma unroll
  for (int p = 0; p < 4; ++p) px_issue(a, L, smem, kt, slot, p);
}

// One direct load per wavefront: the row indices sorted_pos[tseg & ~3 ..]
// (512 entries; past the routed rows they read as zero, readers clamp to the
// segment) into the LDS table; wavefronts w and w + 2 bring the same part.
__device__ __forceinline__ void px_issue_table(const PrefillArgs& a, unsigned char* smem, int tseg) {
  const int lane = threadIdx.x & 63;
  const int half = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 1;
  px_dma16(make_rsrc(a.sorted_pos, (uint32_t)a.rows_total * 4u), 4 * ((tseg & ~3) + 256 * half + 4 * lane), 0,
           smem + kPxTable + 1024 * half);
}

// A wide item's load sources: wavefronts 0..3 bring its 32 activation rows
// (one A load each, as a one-m-block item's); every wavefront the words of
// its 32 tile rows of each n-tile, wavefronts 0..3 the scale chunks of each.
struct PxLoadsW {
  __amdgpu_buffer_rsrc_t wsrc, ssrc;
  int avoff, bstride;
  int bvoff[kPxWide], svoff[kPxWide];
  int na, n;
};

template <int MODE>
__device__ __forceinline__ PxLoadsW px_loads_w(const PrefillArgs& a, const PxItem& it, const unsigned char* smem) {
  PxLoadsW L;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int* table = reinterpret_cast<const int*>(smem + kPxTable);
  const bool areal = wave < 4;
  const int r = 8 * wave + (lane >> 3);
  const int rr = min(r, it.nrows - 1);
  const int64_t src = MODE == kModeGateUp ? (areal ? table[(it.seg0 & 3) + rr] : 0) / a.topk : it.seg0 + rr;
  const int chunk = (lane & 7) ^ ((r >> 1) & 7);
  L.avoff = areal ? (int)(src * a.lda * 2) + 16 * chunk : 0;
  L.na = areal ? 1 : 0;
  L.n = L.na + kPxWide + (wave < 4 ? kPxWide : 0);
  const int K2 = a.K >> 1;
  if (a.wt != nullptr) {
    // tiled copy: n-tiles past the expert's read past the descriptor's range
    // (zeros); their results are not stored
    const int nkt = a.K / kPxKT;
    const int64_t per_e = (int64_t)a.n_nt * nkt * 2048;
    L.wsrc = make_rsrc(reinterpret_cast<const uint32_t*>(a.wt) + (int64_t)it.e * per_e, (uint32_t)(per_e * 4));
#pragma unroll
    for (int b = 0; b < kPxWide; ++b) L.bvoff[b] = (it.nt + b) * nkt * 8192 + wave * 1024 + 16 * lane;
    L.bstride = 8192;
  } else {
    L.wsrc = make_rsrc(reinterpret_cast<const uint32_t*>(a.wp) + (int64_t)it.e * a.N * (a.K >> 3),
                       (uint32_t)a.N * K2);
#pragma unroll
    for (int b = 0; b < kPxWide; ++b)
      L.bvoff[b] = px_weight_row<MODE>(a, it.nt + b, 32 * wave + (lane >> 1)) * K2 + 16 * (lane & 1);
    L.bstride = kPxKT / 2;
  }
  const uintptr_t sbase = reinterpret_cast<uintptr_t>(a.ws + (int64_t)it.e * a.N * a.ng);
  L.ssrc = make_rsrc(reinterpret_cast<const void*>(sbase & ~uintptr_t(15)), (uint32_t)a.N * a.ng * 2u + 16u);
#pragma unroll
  for (int b = 0; b < kPxWide; ++b)
    L.svoff[b] = wave < 4 ? (int)(sbase & 15) + px_weight_row<MODE>(a, it.nt + b, 64 * wave + lane) * a.ng * 2 : 0;
  return L;
}

// Part `part` (0..3, issued before MFMA step `part`) of a wide item's stage
// kt into ring slot `slot`: part 0 the A load, part p < kPxWide the words of
// n-tile p, part p >= 1 the scale chunks of n-tile p - 1.
__device__ __forceinline__ void px_issue_w(const PrefillArgs& a, const PxLoadsW& L, unsigned char* smem, int kt,
                                           int slot, int part) {
  static_assert(kPxWide <= 3, "four parts carry the loads of three n-tiles");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned char* st = smem + slot * kPxStageBytes;
  if (part == 0 && L.na > 0)
    px_dma16(make_rsrc(a.act, (uint32_t)a.act_bytes), L.avoff, kt * (kPxKT * 2), st + wave * 1024);
  if (part < kPxWide) px_dma16(L.wsrc, L.bvoff[part < kPxWide ? part : 0], kt * L.bstride, st + px_wide_b(part) + wave * 1024);
  if (part >= 1 && part <= kPxWide && wave < 4) {
    const int b = part >= 1 ? part - 1 : 0;
    const int gpair = ((kt * kPxKT) >> a.gshift) & ~1;
    px_dma16(L.ssrc, (L.svoff[b] + 2 * gpair) & ~15, 0, st + px_wide_s(b) + 1024 * wave);
  }
}

// Issues an item's stages 0 and 1 into ring slots q0 and q0 + 1; returns the
// wavefront's loads per stage.  Gate_up: the LDS table holds the item's rows.
template <int MODE>
__device__ __forceinline__ int px_issue_first(const PrefillArgs& a, const PxItem& it, unsigned char* smem, int q0) {
  const int q1 = q0 == kPxStages - 1 ? 0 : q0 + 1;
  if (it.nb > 1) {
    const PxLoadsW L = px_loads_w<MODE>(a, it, smem);
#pragma unroll
    for (int p = 0; p < 4; ++p) px_issue_w(a, L, smem, 0, q0, p);
#pragma unroll
    for (int p = 0; p < 4; ++p) px_issue_w(a, L, smem, 1, q1, p);
    return L.n;
  }
  const PxLoads L = px_loads<MODE>(a, it, smem);
  px_issue_all(a, L, smem, 0, q0);
  px_issue_all(a, L, smem, 1, q1);
  return L.n;
}

// Multiply one item.  On entry its stages 0 and 1 are issued into slots p0
// and p0 + 1 (this wavefront's n_inflight loads each; gate_up: the LDS table
// holds the item's rows).  After its last stage it issues the next item's
// stages 0 and 1 (when has_next) and returns their per-stage load count;
// the epilogue runs while they land.
// SPLIT (gate_up's last n-tile when I % 128 == 64: only wavefronts 0..3
// have columns): wavefront w multiplies the weight rows of wavefront w % 4
// with m-blocks MB (w / 4) .. + MB - 1 of the item's 2 MB, so all eight
// wavefronts share the work instead of four idling.
// With fetch_q (non-null) wavefront 0 takes an index from that queue
// counter during the last stage (no stage load is issued after it, so the
// stage's vmcnt(0) wait covers it) and leaves it in LDS at kPxQSlot.
template <int MODE, int MB, bool SPLIT = false>
__device__ __forceinline__ int px_run(const PrefillArgs& a, unsigned char* smem, const PxItem& it,
                                      const PxItem& nx, bool has_next, int p0, int n_inflight,
                                      int* fetch_q) {
  static_assert(!SPLIT || MODE == kModeGateUp, "only gate_up has half n-tiles");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wg = SPLIT ? (wave & 3) : wave;      // weight rows 32 wg .. of the tile
  const int mo = SPLIT ? (wave >> 2) * MB : 0;   // first m-block
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
  for (int s = 0; s < 4; ++s) aoff[s] = mo * 4096 + c * 128 + 16 * ((4 * h + s) ^ ((c >> 1) & 7));
  const int boff = kPxBOff + (32 * wg + c) * 32 + 16 * h;
  // the scale chunk of tile row 32 wave + c; the pair sits at byte
  // (2 (row ng + pair group)) % 16 of it
  const int soff = kPxSOff + (32 * wg + c) * 16;
  const int srow2 = (int)(reinterpret_cast<uintptr_t>(a.ws + (int64_t)it.e * a.N * a.ng) & 15) +
                    px_weight_row<MODE>(a, nt, 32 * wg + c) * a.ng * 2;
  auto soff_of = [&](int t) -> int { return soff + ((srow2 + 2 * (((t * kPxKT) >> gshift) & ~1)) & 15); };
  // wavefronts whose columns lie past the matrix (gate_up's last n-tile
  // when I % 128 == 64) do no MFMA work and store nothing
  const bool work = SPLIT || (MODE == kModeGateUp ? 128 * nt + 16 * wave < a.I : kPxBN * nt + 32 * wave < a.N);

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
  // D[weight row][activation row]: the dequantised weights are the MFMA's A
  // operand, the activation rows its B operand
  auto mfmas = [&](const u32x4_t* af, u32x4_t bf) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma32x(bf, af[mb], acc[mb]);
  };
  auto stage_ptr = [&](int sl) -> const unsigned char* { return smem + sl * kPxStageBytes; };
  // the loads issued after the awaited stage: those of the stage issued in
  // this iteration (n of them)
  auto no_hook = [] {};
  // hook: runs after the wait, before the barrier (its LDS writes are seen
  // by every wavefront after it)
  auto wait_and_sync = [&](int n, auto hook) {
    __builtin_amdgcn_sched_barrier(0);
    px_wait_vm(n);
    __builtin_amdgcn_sched_barrier(0);
    hook();
    px_barrier();
  };

  wait_and_sync(n_inflight, no_hook);  // stage 0 landed (stage 1 may still be loading)
  // Software pipeline: each A fragment register is reloaded with the next
  // step's fragment right after the MFMA that reads it, and the next step's
  // B fragment is dequantised while the current step's MFMAs run.  Stage
  // t's last-step fragments are in registers before the barrier that ends
  // the stage, so after it each MFMA of that step is followed by the read
  // of stage t + 1's first fragment for the same block.
  u32x4_t af[MB];
  u32x4_t bw = {0u, 0u, 0u, 0u};
  float sc = 0.f;
  const ExactRegs kr = exact_regs();
  if (work) {
    read_a(stage_ptr(p0), 0, af);
    bw = *reinterpret_cast<const u32x4_t*>(stage_ptr(p0) + boff);
    sc = scale_of(0, *reinterpret_cast<const uint32_t*>(stage_ptr(p0) + soff_of(0)));
  }
  int slot = p0;
  int slot2 = p0 + 2 >= kPxStages ? p0 + 2 - kPxStages : p0 + 2;
  // one k stage: refill the slot stage t - 1 used (issue(slot2)), multiply
  // stage t, wait for stage t + 1 and meet the other wavefronts
  auto iter = [&](int t, int n, auto issue, auto hook) {
    const int nslot = slot == kPxStages - 1 ? 0 : slot + 1;
    if (work) {
      const unsigned char* st = stage_ptr(slot);
      const ExactScale es = exact_scale(sc);
      const uint32_t wv[4] = {bw.x, bw.y, bw.z, bw.w};
      u32x4_t bf = unpack_exact<false>(wv[0], es, kr);
#pragma unroll
      for (int s2 = 0; s2 < 3; ++s2) {
        issue(slot2, s2);
        const u32x4_t bfn = unpack_exact<false>(wv[s2 + 1], es, kr);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          acc[mb] = mfma32x(bf, af[mb], acc[mb]);
          af[mb] = *reinterpret_cast<const u32x4_t*>(st + mb * 4096 + aoff[s2 + 1]);
        }
        bf = bfn;
      }
      issue(slot2, 3);
      wait_and_sync(n, hook);  // stage t + 1 landed (stage t + 2 may still be loading)
      if (t + 1 < nkt) {
        const unsigned char* sn = stage_ptr(nslot);
        bw = *reinterpret_cast<const u32x4_t*>(sn + boff);
        const uint32_t sp = *reinterpret_cast<const uint32_t*>(sn + soff_of(t + 1));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          acc[mb] = mfma32x(bf, af[mb], acc[mb]);
          af[mb] = *reinterpret_cast<const u32x4_t*>(sn + mb * 4096 + aoff[0]);
        }
        sc = scale_of(t + 1, sp);
      } else {
        mfmas(af, bf);
      }
    } else {
#pragma unroll
      for (int p = 0; p < 4; ++p) issue(slot2, p);
      wait_and_sync(n, hook);
    }
    slot = nslot;
    slot2 = slot2 == kPxStages - 1 ? 0 : slot2 + 1;
  };
  {
    const PxLoads lc = px_loads<MODE>(a, it, smem);
    for (int t = 0; t + 2 < nkt; ++t)
      iter(t, lc.n, [&](int sl, int p) { px_issue(a, lc, smem, t + 2, sl, p); }, no_hook);
  }
  // the last two stages issue no stage loads; the second-to-last brings the
  // row-index table (gate_up: the next item's rows, for its load sources;
  // down: this item's output rows, for its epilogue)
  const int tseg = MODE == kModeGateUp ? (has_next ? nx.seg0 : seg0) : seg0;
  iter(nkt - 2, 1, [&](int, int p) {
    if (p == 0) px_issue_table(a, smem, tseg);
  }, no_hook);
  const bool fetch = fetch_q != nullptr && wave == 0;  // wavefront-uniform
  int fv = 0;
  iter(nkt - 1, 0,
       [&](int, int p) {
         if (p == 0 && fetch && lane == 0) fv = __hip_atomic_fetch_add(fetch_q, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
       },
       [&] {
         if (fetch && lane == 0) *reinterpret_cast<int*>(smem + kPxQSlot) = fv;
       });
  // every wavefront is past the last barrier: the next item's first two
  // stages go into the slots of this item's stages nkt - 3 and nkt - 2
  const int n_next = has_next ? px_issue_first<MODE>(a, nx, smem, (p0 + nkt) % kPxStages) : 0;
  if (!work) return n_next;

  // ---- epilogue.  Lane l holds, for activation row 32 mb + c of block mb,
  // the wavefront's weight rows 8 J + 4 h + i in acc[mb][4 J + i] (J, i =
  // 0..3): four consecutive output columns per J.  gate_up stores them as 8
  // bytes from registers: weight rows 0..15 are the gate rows and 16..31
  // their up rows, so acc[mb][q] (gate) pairs with acc[mb][q + 8] (up).
#pragma unroll
  for (int mb = 0; mb < MB && MODE == kModeGateUp; ++mb) {
    const int grow = 32 * (mo + mb) + c;
    if (grow >= nrows) continue;
    {
      uint16_t* orow = a.out + (int64_t)(seg0 + grow) * a.ldo + 128 * nt + 16 * wg + 4 * h;
#pragma unroll
      for (int J = 0; J < 2; ++J) {
        float hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g = round_bf16(acc[mb][4 * J + i]);
          const float u = round_bf16(acc[mb][4 * J + i + 8]);
          hv[i] = round_bf16(gelu_tanh_f32(g)) * u;
        }
        *reinterpret_cast<uint2*>(orow + 8 * J) = make_uint2(pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3]));
      }
    }
  }
  if (MODE == kModeDown) {
    // dn rows are long (N columns, rows scattered by sorted_pos): the
    // wavefront's 32 columns of each row go out as 16-byte stores, through
    // LDS one m-block at a time (it reads only what it wrote: no barrier)
    const int* table = reinterpret_cast<const int*>(smem + kPxTable);
    unsigned char* ob = smem + kPxEpiOff + wave * kPxEpiBytes;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int J = 0; J < 4; ++J)
        *reinterpret_cast<uint2*>(ob + c * kPxEpiPitch + 2 * (8 * J + 4 * h)) =
            make_uint2(pack_bf16x2(acc[mb][4 * J], acc[mb][4 * J + 1]), pack_bf16x2(acc[mb][4 * J + 2], acc[mb][4 * J + 3]));
#pragma unroll
      for (int itr = 0; itr < 2; ++itr) {
        const int idx = lane + 64 * itr;
        const int row = idx >> 2, q4 = idx & 3;
        const int grow = 32 * mb + row;
        if (grow < nrows) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ob + row * kPxEpiPitch + 16 * q4);
          st16(a.out + (int64_t)table[(seg0 & 3) + grow] * a.N + kPxBN * nt + 32 * wave + 8 * q4, v);
        }
      }
    }
  }
  return n_next;
}

// Multiply one wide item (kPxWide n-tiles of a tail of at most 32 rows), in
// px_run's stage protocol.  Each n-tile's outputs are px_run<MODE, 1>'s for
// that n-tile bit for bit: the same MFMA on the same operands, one k step
// after the other.
template <int MODE>
__device__ __forceinline__ int px_run_w(const PrefillArgs& a, unsigned char* smem, const PxItem& it,
                                        const PxItem& nx, bool has_next, int p0, int n_inflight,
                                        int* fetch_q) {
  constexpr int NB = kPxWide;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nkt = a.K / kPxKT;
  const int h = lane >> 5;
  const int c = lane & 31;
  const int gshift = a.gshift;
  const int nt0 = it.nt, seg0 = it.seg0, nrows = it.nrows;

  int aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = c * 128 + 16 * ((4 * h + s) ^ ((c >> 1) & 7));
  int boff[NB], soffb[NB], srow2[NB];
  const int sb15 = (int)(reinterpret_cast<uintptr_t>(a.ws + (int64_t)it.e * a.N * a.ng) & 15);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    boff[b] = px_wide_b(b) + (32 * wave + c) * 32 + 16 * h;
    soffb[b] = px_wide_s(b) + (32 * wave + c) * 16;
    srow2[b] = sb15 + px_weight_row<MODE>(a, nt0 + b, 32 * wave + c) * a.ng * 2;
  }
  f32x16_t acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[b][q] = 0.f;
  auto scale_of = [&](int t, uint32_t sp) -> float {
    const int g = (t * kPxKT + 32 * h) >> gshift;
    const int sel = g - (((t * kPxKT) >> gshift) & ~1);  // 0 or 1
    return bf16_bits_to_f32((sp >> (16 * sel)) & 0xFFFFu);
  };
  auto stage_ptr = [&](int sl) -> const unsigned char* { return smem + sl * kPxStageBytes; };
  auto no_hook = [] {};
  auto wait_and_sync = [&](int n, auto hook) {
    __builtin_amdgcn_sched_barrier(0);
    px_wait_vm(n);
    __builtin_amdgcn_sched_barrier(0);
    hook();
    px_barrier();
  };
  const ExactRegs kr = exact_regs();

  wait_and_sync(n_inflight, no_hook);  // stage 0 landed
  int slot = p0;
  int slot2 = p0 + 2 >= kPxStages ? p0 + 2 - kPxStages : p0 + 2;
  // one k stage: read its words and scales, refill the slot stage t - 1 used
  // (issue(slot2)) while multiplying, wait for stage t + 1 and meet
  auto iter = [&](int t, int n, auto issue, auto hook) {
    const unsigned char* st = stage_ptr(slot);
    u32x4_t bw[NB];
    ExactScale es[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      bw[b] = *reinterpret_cast<const u32x4_t*>(st + boff[b]);
      const int so = soffb[b] + ((srow2[b] + 2 * (((t * kPxKT) >> gshift) & ~1)) & 15);
      es[b] = exact_scale(scale_of(t, *reinterpret_cast<const uint32_t*>(st + so)));
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      issue(slot2, s);
      const u32x4_t af = *reinterpret_cast<const u32x4_t*>(st + aoff[s]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t w = s == 0 ? bw[b].x : s == 1 ? bw[b].y : s == 2 ? bw[b].z : bw[b].w;
        acc[b] = mfma32x(unpack_exact<false>(w, es[b], kr), af, acc[b]);
      }
    }
    wait_and_sync(n, hook);  // stage t + 1 landed (stage t + 2 may still be loading)
    slot = slot == kPxStages - 1 ? 0 : slot + 1;
    slot2 = slot2 == kPxStages - 1 ? 0 : slot2 + 1;
  };
  {
    const PxLoadsW lc = px_loads_w<MODE>(a, it, smem);
    for (int t = 0; t + 2 < nkt; ++t)
      iter(t, lc.n, [&](int sl, int p) { px_issue_w(a, lc, smem, t + 2, sl, p); }, no_hook);
  }
  const int tseg = MODE == kModeGateUp ? (has_next ? nx.seg0 : seg0) : seg0;
  iter(nkt - 2, 1, [&](int, int p) {
    if (p == 0) px_issue_table(a, smem, tseg);
  }, no_hook);
  const bool fetch = fetch_q != nullptr && wave == 0;  // wavefront-uniform
  int fv = 0;
  iter(nkt - 1, 0,
       [&](int, int p) {
         if (p == 0 && fetch && lane == 0) fv = __hip_atomic_fetch_add(fetch_q, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
       },
       [&] {
         if (fetch && lane == 0) *reinterpret_cast<int*>(smem + kPxQSlot) = fv;
       });
  const int n_next = has_next ? px_issue_first<MODE>(a, nx, smem, (p0 + nkt) % kPxStages) : 0;

  // epilogue per n-tile, as px_run's for m-block 0 (n-tiles past the
  // matrix, and gate_up columns past I, store nothing)
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int nt = nt0 + b;
    if (MODE == kModeGateUp) {
      if (128 * nt + 16 * wave < a.I && c < nrows) {
        uint16_t* orow = a.out + (int64_t)(seg0 + c) * a.ldo + 128 * nt + 16 * wave + 4 * h;
#pragma unroll
        for (int J = 0; J < 2; ++J) {
          float hv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = round_bf16(acc[b][4 * J + i]);
            const float u = round_bf16(acc[b][4 * J + i + 8]);
            hv[i] = round_bf16(gelu_tanh_f32(g)) * u;
          }
          *reinterpret_cast<uint2*>(orow + 8 * J) = make_uint2(pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3]));
        }
      }
    } else if (kPxBN * nt + 32 * wave < a.N) {
      const int* table = reinterpret_cast<const int*>(smem + kPxTable);
      unsigned char* ob = smem + kPxEpiOff + wave * kPxEpiBytes;
#pragma unroll
      for (int J = 0; J < 4; ++J)
        *reinterpret_cast<uint2*>(ob + c * kPxEpiPitch + 2 * (8 * J + 4 * h)) =
            make_uint2(pack_bf16x2(acc[b][4 * J], acc[b][4 * J + 1]), pack_bf16x2(acc[b][4 * J + 2], acc[b][4 * J + 3]));
#pragma unroll
      for (int itr = 0; itr < 2; ++itr) {
        const int idx = lane + 64 * itr;
        const int row = idx >> 2, q4 = idx & 3;
        if (row < nrows) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ob + row * kPxEpiPitch + 16 * q4);
          st16(a.out + (int64_t)table[(seg0 & 3) + row] * a.N + kPxBN * nt + 32 * wave + 8 * q4, v);
        }
      }
    }
  }
  return n_next;
}

template <int MODE>
__device__ __forceinline__ int px_dispatch(const PrefillArgs& a, unsigned char* smem, const PxItem& it,
                                           const PxItem& nx, bool has_next, int p0, int n_inflight,
                                           int* fetch_q) {
  if (it.nb > 1) return px_run_w<MODE>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
  if constexpr (MODE == kModeGateUp) {
    if (a.I - 128 * it.nt == 64 && it.mb >= 2) {
      // half n-tile: eight wavefronts on four wavefronts' columns
      if (it.mb == 8) return px_run<MODE, 4, true>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
      if (it.mb == 4) return px_run<MODE, 2, true>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
      return px_run<MODE, 1, true>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
    }
  }
  if (it.mb == 8) return px_run<MODE, 8>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
  if (it.mb == 4) return px_run<MODE, 4>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
  if (it.mb == 2) return px_run<MODE, 2>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
  return px_run<MODE, 1>(a, smem, it, nx, has_next, p0, n_inflight, fetch_q);
}

// Persistent grid, one workgroup per CU.  down: local item i of XCD x is
// n-tile i % n_nt of the XCD's m-tile i / n_nt, tile list entry x + 8 (i /
// n_nt), so an m-tile's activation rows are read into one L2 for its 11
// n-tiles; workgroup b of XCD x = b % 8 takes local items b / 8 and b / 8 +
// P (P = workgroups per XCD), then the items that XCD's queue counter
// (queues[x]) hands out, 2 P, 2 P + 1, ...  gate_up: item i is n-tile i %
// n_nt of tile list entry i / n_nt, workgroup b takes items b and b + P (P
// = all workgroups), then those of the one queue (queues[0]): its items
// differ more in cost (segment tails, the half n-tile) and the XCDs in
// speed, and the whole chip draining one queue ends them closer together
// than the rows kept in one L2 save.  The list runs from large tiles to
// small, so large items go first.  Workgroups ask in the order they get
// there, during the last stage of the item before their next one, so the
// index is known one item ahead (the next item's rows and first stages are
// loaded during the current one).  queues[8] counts the workgroups that
// have left; the expert sort zeroes the counters and the last workgroup to
// leave resets them.  Without queues the deal is fixed: items b + r P.
template <int MODE>
__global__ __launch_bounds__(kPxThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_prefill_x(PrefillArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int ntiles = ld_uniform(a.counters, 1);
  const int tiny0 = ld_uniform(a.counters, 2), tiny1 = ld_uniform(a.counters, 3);  // the smallest tails
  constexpr bool kChip = MODE == kModeGateUp;  // one queue for the chip
  const int x0 = kChip ? 0 : (int)(blockIdx.x & 7);
  const int xs = kChip ? 1 : 8;
  const int n_local = kChip ? ntiles : (ntiles > x0 ? (ntiles - x0 + 7) >> 3 : 0);  // the queue's m-tiles
  // the queue's m-tiles before list entry b
  auto local = [&](int b) { return kChip ? b : (b > x0 ? (b - x0 + 7) >> 3 : 0); };
  const int t0 = local(tiny0), t1 = local(tiny1);
  const int n_wide = (a.n_nt + kPxWide - 1) / kPxWide;
  const int it_end = (n_local - (t1 - t0)) * a.n_nt + (t1 - t0) * n_wide;
  const int P = kChip ? (int)gridDim.x : (int)(gridDim.x >> 3);
  int* const queue = a.queues != nullptr ? a.queues + x0 : nullptr;
  // the last workgroup to leave resets the counters for the next launch
  // (every other one has taken its last index before counting itself out)
  auto leave = [&] {
    if (a.queues == nullptr || threadIdx.x != 0) return;
    const int d = __hip_atomic_fetch_add(a.queues + 8, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == (int)gridDim.x - 1) {
#pragma unroll
      for (int x = 0; x < 9; ++x) __hip_atomic_store(a.queues + x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  int item = kChip ? (int)blockIdx.x : (int)(blockIdx.x >> 3);
  if (item >= it_end) {
    leave();
    return;
  }
  const int nkt = a.K / kPxKT;
  PxItem cur = px_item_info(a, x0, xs, t0, t1, n_wide, item);
  if (MODE == kModeGateUp) {
    // the first item's gathered rows into the table (nothing else in flight)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t tsrc = make_rsrc(a.sorted_pos, (uint32_t)a.rows_total * 4u);
    if (wave < 2) px_dma16(tsrc, 4 * ((cur.seg0 & ~3) + 256 * wave + 4 * lane), 0, smem + kPxTable + 1024 * wave);
    __builtin_amdgcn_s_waitcnt(px_vm_wait(0));
    px_barrier();
  }
  int n_inflight = px_issue_first<MODE>(a, cur, smem, 0);
  int p0 = 0;
  int nitem = item + P;
  for (;;) {
    const bool has_next = nitem < it_end;
    const PxItem nxt = has_next ? px_item_info(a, x0, xs, t0, t1, n_wide, nitem) : cur;
    // with a next item, take the index of the one after it during this item
    n_inflight = px_dispatch<MODE>(a, smem, cur, nxt, has_next, p0, n_inflight, has_next ? queue : nullptr);
    if (!has_next) break;
    item = nitem;
    nitem = queue != nullptr ? 2 * P + __builtin_amdgcn_readfirstlane(*reinterpret_cast<volatile int*>(smem + kPxQSlot))
                             : item + P;
    cur = nxt;
    p0 = (p0 + nkt) % kPxStages;
  }
  // the loads issued past the last stage land before the workgroup leaves
  __builtin_amdgcn_s_waitcnt(px_vm_wait(0));
  leave();
}

// The tiled weight copy: piece (e, nt, kt, tr, h) = 16 bytes of weight row
// px_weight_row(nt, tr) at byte 32 kt + 16 h, so stage kt of n-tile nt is
// 8 KiB in the order the kernel's B loads fill LDS (tile row tr at 32 tr).
template <int MODE>
__global__ __launch_bounds__(256) void k_tile_prefill(const uint32_t* __restrict__ packed,
                                                      uint32_t* __restrict__ tiled, PrefillArgs a,
                                                      int64_t pieces) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= pieces) return;
  const int nkt = a.K / kPxKT;
  const int h = (int)(p & 1);
  const int tr = (int)((p >> 1) & 255);
  int64_t q = p >> 9;
  const int kt = (int)(q % nkt);
  q /= nkt;
  const int nt = (int)(q % a.n_nt);
  const int64_t e = q / a.n_nt;
  const int row = px_weight_row<MODE>(a, nt, tr);
  const int64_t src = (e * a.N + row) * (int64_t)(a.K / 2) + 32 * kt + 16 * h;
  *reinterpret_cast<u32x4_t*>(tiled + p * 4) = *reinterpret_cast<const u32x4_t*>(packed + src / 4);
}

size_t prefill_tiled_bytes_per_expert(int mode, int64_t H, int64_t I) {
  if (H % kPxKT != 0 || I % kPxKT != 0 || H < 3 * kPxKT || I < 3 * kPxKT) return 0;
  const int64_t K = mode == kModeGateUp ? H : I;
  const int64_t n_nt = mode == kModeGateUp ? (I + 127) / 128 : (H + 255) / 256;
  return (size_t)(n_nt * (K / kPxKT) * 8192);
}

hipError_t launch_tile_prefill(int mode, const int32_t* packed, int E, int H, int I, int32_t* tiled,
                               hipStream_t s) {
  if (prefill_tiled_bytes_per_expert(mode, H, I) == 0) return hipErrorInvalidValue;
  PrefillArgs a{};
  a.I = I;
  a.N = mode == kModeGateUp ? 2 * I : H;
  a.K = mode == kModeGateUp ? H : I;
  a.n_nt = mode == kModeGateUp ? (I + 127) / 128 : (H + 255) / 256;
  const int64_t pieces = (int64_t)E * a.n_nt * (a.K / kPxKT) * 512;
  if (pieces == 0) return hipSuccess;
  const dim3 grid((unsigned)((pieces + 255) / 256));
  const uint32_t* src = reinterpret_cast<const uint32_t*>(packed);
  uint32_t* dst = reinterpret_cast<uint32_t*>(tiled);
  if (mode == kModeGateUp)
    hipLaunchKernelGGL(k_tile_prefill<kModeGateUp>, grid, dim3(256), 0, s, src, dst, a, pieces);
  else
    hipLaunchKernelGGL(k_tile_prefill<kModeDown>, grid, dim3(256), 0, s, src, dst, a, pieces);
  return hipGetLastError();
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

size_t prefill_x_lds_bytes() { return (size_t)kPxLds; }

// H and I multiples of the 64-wide stage, at least three stages; G a power of two >= 32 whose
// group counts per row are even for both matrices (a stage's scale pair is
// one aligned dword)
bool prefill_x_supported(int64_t H, int64_t I, int64_t G) {
  if (H % kPxKT != 0 || I % kPxKT != 0 || H < 3 * kPxKT || I < 3 * kPxKT || G < 32 || (G & (G - 1)) != 0)
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
