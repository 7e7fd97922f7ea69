// Prefill-shaped W4A16 MoE expert GEMMs (many rows per expert).
//
//   MODE = gateup : inter[s] = gelu(x[tok(s)] Wg^T) * (x[tok(s)] Wu^T)
//                   (quantization.py:112-120), rows s in expert-segment order
//   MODE = down   : dn[sorted_pos[s]] = inter[s] W_d^T   (quantization.py:122-127)
//
// Work item = (m-tile of one expert's segment, n-tile of kPfBN weight rows).
// The sort produces the m-tile list; items are spread over a persistent grid
// so that each XCD (own L2) walks one contiguous run of items: the n-tiles of
// one m-tile share its activation rows, consecutive m-tiles of one expert
// share its weights.
//
// Per K stage (kPfBK = 64) the workgroup stages
//   A: BM activation rows x 64 k, bf16, gathered by row;
//   B: 128 weight rows x 64 k, unpacked once per workgroup with the exact
//      dequantisation bf16_RNE(q * s) (bit-identical to dequantize_int4_packed)
// into LDS in MFMA fragment order, so every fragment read is one contiguous
// 1 KiB ds_read_b128 per wavefront.  Four wavefronts (2 x 2) each own a
// (BM/2) x 64 sub-tile of v_mfma_f32_16x16x32_bf16 accumulators (fp32).
// Loads for stage s+1 are in flight while stage s is multiplied.
#include "common.hpp"
#include "launch.hpp"

namespace w4a16 {

namespace {

constexpr int kPfThreads = 256;
constexpr int kPfBK = 64;
// K stages of global loads in flight (register slots)
constexpr int kPfDepth = 3;

// B tile columns -> MFMA column blocks.  gate_up: tile columns 0..63 are gate
// rows j0..j0+63, 64..127 the up rows I+j0..; wavefront wn multiplies gate
// blocks 2wn, 2wn+1 and the matching up blocks 4+2wn, 5+2wn so the epilogue
// finds gate and up values in one lane.
template <int MODE>
__device__ __forceinline__ int col_block(int wn, int fn) {
  if (MODE == kModeGateUp) return fn < 2 ? 2 * wn + fn : 4 + 2 * wn + (fn - 2);
  return 4 * wn + fn;
}

}  // namespace

template <int MODE, int BM>
__global__ __launch_bounds__(kPfThreads) void k_prefill(PrefillArgs a) {
  constexpr int FM = BM / 32;       // 16-row fragments per wavefront
  constexpr int FN = 4;             // 16-column fragments per wavefront
  constexpr int AR = BM / 32;       // A rows each thread stages (one 16-byte chunk each)
  constexpr int A_PITCH = 9;        // 16-byte slots per A row: 8 chunks + 1 pad
  constexpr int A_SLOTS = BM * A_PITCH;
  constexpr int B_SLOTS = kPfBN * 8;
  constexpr int STAGE = A_SLOTS + B_SLOTS;
  constexpr int D = kPfDepth;
  extern __shared__ u32x4_t lds[];  // 2 * STAGE slots (prefill_lds_bytes)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  const int K = a.K;
  const int K8 = K >> 3;
  const int nks = K / kPfBK;
  const int ntiles = a.counters[1];
  const int total = ntiles * a.n_nt;
  // XCD-contiguous item ranges (workgroups are dealt to the 8 XCDs in turn)
  const int nb = gridDim.x;
  const int xcd = blockIdx.x & 7;
  const int per_xcd = nb >> 3;
  const int chunk = (total + 7) >> 3;
  const int it_end = min(total, (xcd + 1) * chunk);

  // Staging roles:
  //  A: rows (tid >> 3) + 32 i, 16-byte chunk tid & 7 -- one load instruction
  //     reads 8 whole 128-byte row segments; rows sit in LDS at a pitch of 144
  //     bytes, so both these stores and the fragment reads below (lane l: row
  //     l % 16, chunk l / 16) touch distinct banks;
  //  B: tile column (tid & 15) + 16 (tid >> 5), k half (tid >> 4) & 1, stored
  //     in fragment order (each store instruction covers 1 KiB contiguously).
  const int ar0 = tid >> 3, ac = tid & 7;
  const int bn = (tid & 15) + 16 * (tid >> 5);
  const int bh = (tid >> 4) & 1;
  const ExactRegs kr = exact_regs();

  for (int item = xcd * chunk + (blockIdx.x >> 3); item < it_end; item += per_xcd) {
    const int mt = item / a.n_nt;
    const int nt = item - mt * a.n_nt;
    const int tile = a.tiles[mt];
    const int e = tile >> 16;
    const int seg0 = a.offsets[e] + (tile & 0xFFFF) * BM;
    const int nrows = min(BM, a.offsets[e + 1] - seg0);

    // activation row sources (rows past the segment repeat its last row;
    // their results are never stored)
    const uint16_t* arow[AR];
#pragma unroll
    for (int i = 0; i < AR; ++i) {
      const int rr = min(ar0 + 32 * i, nrows - 1);
      if (MODE == kModeGateUp) {
        const int tok = a.sorted_pos[seg0 + rr] / a.topk;
        arow[i] = a.act + (int64_t)tok * K + ac * 8;
      } else {
        arow[i] = a.act + (int64_t)(seg0 + rr) * K + ac * 8;
      }
    }
    // 16-row fragments of this wavefront that hold real rows: MFMA work on
    // fragments made only of padding rows is skipped
    const int nvf = __builtin_amdgcn_readfirstlane(
        max(0, min(FM, (nrows - wm * (BM / 2) + 15) >> 4)));
    int ncol;
    if (MODE == kModeGateUp)
      ncol = bn < 64 ? nt * 64 + bn : a.I + nt * 64 + (bn - 64);
    else
      ncol = nt * kPfBN + bn;
    const int64_t wrow = (int64_t)e * a.N + ncol;
    const int32_t* wsrc = a.wp + wrow * K8 + 4 * bh;
    const uint16_t* ssrc = a.ws + wrow * a.ng;

    u32x4_t ra[D][AR];
    u32x4_t rw[D];
    uint16_t rs[D];
    auto load_stage = [&](int slot, int ks) {
#pragma unroll
      for (int i = 0; i < AR; ++i) ra[slot][i] = ld16(arow[i] + ks * kPfBK);
      rw[slot] = ld16(wsrc + ks * 8);
      rs[slot] = ssrc[(ks * kPfBK + 32 * bh) / a.G];
    };
    auto store_stage = [&](int buf, int slot) {
      u32x4_t* base = lds + buf * STAGE;
#pragma unroll
      for (int i = 0; i < AR; ++i) base[(ar0 + 32 * i) * A_PITCH + ac] = ra[slot][i];
      const ExactScale es = exact_scale(bf16_bits_to_f32(rs[slot]));
      u32x4_t* bb = base + A_SLOTS + (((bn >> 4) << 1) + bh) * 64 + (bn & 15);
      bb[0] = unpack_exact<false>(rw[slot].x, es, kr);
      bb[16] = unpack_exact<false>(rw[slot].y, es, kr);
      bb[32] = unpack_exact<false>(rw[slot].z, es, kr);
      bb[48] = unpack_exact<false>(rw[slot].w, es, kr);
    };

    f32x4_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf) {
      const u32x4_t* base = lds + buf * STAGE;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4_t af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          if (i < nvf)
            af[i] = base[((wm * FM + i) * 16 + (lane & 15)) * A_PITCH + 4 * h + (lane >> 4)];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bf[j] = base[A_SLOTS + (col_block<MODE>(wn, j) * 2 + h) * 64 + lane];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          if (i < nvf) {
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
          }
      }
    };

    __syncthreads();  // the previous item's epilogue is done with LDS
#pragma unroll
    for (int d = 0; d < D; ++d) load_stage(d, min(d, nks - 1));
    store_stage(0, 0);
    __syncthreads();
    // stage s: register slot s % D holds its loads (already in LDS buffer
    // s & 1); it is refilled with stage s + D, then stage s + 1 (slot
    // (s + 1) % D) is unpacked into the other buffer while s multiplies.
    // Stages past the end load the last stage again (in bounds, unused).
    for (int ks = 0; ks < nks; ks += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const int s = ks + u;
        if (s < nks) {
          load_stage(u, min(s + D, nks - 1));
          compute(s & 1);
          store_stage((s + 1) & 1, (u + 1) % D);
          __syncthreads();
        }
      }
    }

    // epilogue: bf16 results -> wavefront-private LDS rows -> 16-byte stores
    constexpr int OC = MODE == kModeGateUp ? 32 : 64;  // output columns per wavefront
    constexpr int PITCH = OC + 8;                      // bf16 per LDS row (16-byte multiple)
    uint16_t* ob = reinterpret_cast<uint16_t*>(lds) + wave * (BM / 2) * PITCH;
    const int kb = lane >> 4, j16 = lane & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 16 * i + 4 * kb + q;
        if (MODE == kModeGateUp) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float gate = round_bf16(acc[i][j][q]);
            const float act = round_bf16(gelu_tanh_f32(gate));
            const float h = act * round_bf16(acc[i][j + 2][q]);
            ob[r * PITCH + 16 * j + j16] = f32_to_bf16_bits(h);
          }
        } else {
#pragma unroll
          for (int j = 0; j < FN; ++j) ob[r * PITCH + 16 * j + j16] = f32_to_bf16_bits(acc[i][j][q]);
        }
      }
    }
    // the wavefront reads back only what it wrote: LDS ordering within a
    // wavefront needs no barrier
    constexpr int CPR = OC / 8;                  // 16-byte chunks per row
    constexpr int NCH = (BM / 2) * CPR / 64;     // chunks per lane
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int idx = lane + 64 * c;
      const int r = idx / CPR, cc = idx - r * CPR;
      const int row = wm * (BM / 2) + r;
      if (row < nrows) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ob + r * PITCH + 8 * cc);
        if (MODE == kModeGateUp) {
          st16(a.out + (int64_t)(seg0 + row) * a.I + nt * 64 + 32 * wn + 8 * cc, v);
        } else {
          const int64_t orow = a.sorted_pos[seg0 + row];
          st16(a.out + orow * a.N + nt * kPfBN + 64 * wn + 8 * cc, v);
        }
      }
    }
  }
}

size_t prefill_lds_bytes(int BM) {
  return (size_t)2 * (BM * 9 + kPfBN * 8) * 16;
}

// persistent grid: the workgroups that fit on the device at once (a multiple
// of the 8 XCDs), at most one per item
template <typename Kern>
int prefill_grid(Kern kern, size_t lds, int max_items) {
  int dev = 0, cus = 256, per_cu = 1;
  hipDeviceProp_t p;
  if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess &&
      p.multiProcessorCount > 0)
    cus = p.multiProcessorCount;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kPfThreads, lds) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  int g = cus * per_cu;
  if (max_items < g) g = max_items;
  return ((g + 7) / 8) * 8;
}

hipError_t launch_prefill(int mode, PrefillArgs a, int max_mtiles, hipStream_t s) {
  if (max_mtiles <= 0) return hipSuccess;
  const size_t lds = prefill_lds_bytes(kPrefillBM);
  if (mode == kModeGateUp) {
    auto kern = k_prefill<kModeGateUp, kPrefillBM>;
    hipLaunchKernelGGL(kern, dim3(prefill_grid(kern, lds, max_mtiles * a.n_nt)), dim3(kPfThreads),
                       lds, s, a);
  } else {
    auto kern = k_prefill<kModeDown, kPrefillBM>;
    hipLaunchKernelGGL(kern, dim3(prefill_grid(kern, lds, max_mtiles * a.n_nt)), dim3(kPfThreads),
                       lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace w4a16
