// Internal launch interface between the C-ABI layer (capi.hip) and the
// kernel translation units.  Every launcher is asynchronous on `stream` and
// returns hipSuccess or the launch error.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w4a16 {

constexpr int kMaxExperts = 512;
constexpr int kMaxTopK = 32;
// m-tile (token rows) and n-tile (weight rows) of the prefill grouped GEMM
constexpr int kPrefillBM = 128;
constexpr int kPfBN = 128;
// m-tile of the exact-form prefill GEMM (kernels_prefill_x.hip)
constexpr int kPrefillXBM = 256;
// segment tails of at most this many rows (one 32-row MFMA block) are listed
// apart, and the exact-form prefill GEMM takes them three n-tiles per item
constexpr int kPrefillTinyRows = 32;
// prefill work-queue counters in the MoE workspace: gate_up [0, 16), down [16, 32)
constexpr int kPrefillQueueInts = 32;

// One-workgroup top-k + expert sort of the decode router's K-split partials
// (M * topk <= 64): the routing outputs and the plan it writes.
struct TopkSortArgs {
  const float* partial;
  const uint16_t* pes;
  int64_t* idx_out;
  float* w_out;
  int M, E, topk;
  int32_t *sorted_pos, *offsets, *desc, *counters, *tiles;
  int BM, slot_rows;
};

// The decode gate_up launch's own plan (k_decode's SELF): none (it reads the
// plan), kSelfRoute (one token: it also routes), kSelfPlan (it sorts a
// finished top-k itself).
enum DecodeSelf { kSelfNone = 0, kSelfRoute = 1, kSelfPlan = 2 };

// Arguments of the decode-shaped (few rows per weight matrix) MFMA kernel.
struct DecodeArgs {
  const uint16_t* act;        // activation rows (bf16), row length K
  const int32_t* wp;          // packed weights [E?, N, K/8]
  const uint16_t* ws;         // bf16 scales [E?, N, ng]
  const uint16_t* bias;       // dense only, nullable, [N]
  uint16_t* out;              // output rows
  const int32_t* sorted_pos;  // MoE: [M*k] rows t*k+j in expert-segment order
  const int32_t* desc;        // MoE: [E][4] (expert, segment start, rows, 0) per active slot
  const int32_t* n_active;    // MoE: [1]
  int M;     // dense: activation rows
  int N;     // weight rows per expert
  int K;     // reduction length
  int G;     // group size
  int ng;    // ceil(K / G)
  int topk;  // MoE k
  int I;     // gate_up: intermediate size (N / 2)
  int rb;    // activation rows staged in LDS per pass (<= 16)
  int n_ct;  // work items (column tiles) per expert
  int rows_hint;    // most activation rows one expert can have (set by the caller)
  int cg;           // column groups of 16 weight rows per item (set by the launcher)
  int ct_blocks;    // tiled: (item, wavefront) blocks per expert in the copy
  // set by the launcher: the likeliest number of active slots (MoE) and the
  // slot arithmetic for it (workgroups per slot, its division magic, items
  // per workgroup)
  int u_guess, wps_guess, per_guess;
  uint32_t slot_magic;
  // the gate_up launch's own plan (launch_decode's self_args / self_mode):
  // the top-k + sort's arguments (kSelfPlan: idx_out is the finished top-k
  // it reads), the plan written by the launch's last workgroup, and
  // floor(2^32 / M) + 1 (k-major position -> slot j, exact below 2^16)
  TopkSortArgs route;
  uint32_t plan_m_magic;
};

// Arguments of the prefill-shaped grouped GEMM (kernels_prefill.hip).
struct PrefillArgs {
  const uint16_t* act;        // gate_up: hidden [M, K]; down: inter [M*k, K] in segment order
  const int32_t* wp;          // packed weights [E, N, K/8]
  const uint16_t* ws;         // bf16 scales [E, N, ng]
  uint16_t* out;              // gate_up: inter [M*k, I]; down: dn rows t*k+j [M*k, N]
  const int32_t* sorted_pos;  // [M*k] rows t*k+j in expert-segment order
  const int32_t* offsets;     // [E+1] segment starts
  const int32_t* tiles;       // m-tiles (expert << 16 | tile index in the segment)
  const int32_t* counters;    // [1] = number of m-tiles, [2] / [3] = start / end of the tails of <= kPrefillTinyRows rows
  int N, K, G, ng, topk, I;
  int n_nt;                   // n-tiles per m-tile
  // exact-form kernel: row strides (elements) of act and of the gate_up output
  int lda, ldo;
  // the work queues of this launch, 9 ints (one counter per XCD, then the
  // count of workgroups that have left), zero at launch
  int32_t* queues;
  // exact-form kernel: bytes of act (its buffer bound), log2 G and the
  // routed rows (entries of sorted_pos)
  int64_t act_bytes;
  int gshift;
  int rows_total;
  // exact-form kernel, nullable: the weights' tiled copy (k_tile_prefill):
  // [E][n_nt][K/64][256 tile rows][32 B], each item's stage one 8 KiB block
  const int32_t* wt;
};

enum DecodeMode { kModeDense = 0, kModeGateUp = 1, kModeDown = 2 };

// Arguments of the fused down projection + weighted combine for decode
// sizes (kernels_down_combine.hip).
constexpr int kDownCombineMaxRows = 64;
struct DownCombineArgs {
  const uint16_t* act;        // intermediate rows [M*k, K] in segment order
  const int32_t* wp;          // packed down weights [E, N, K/8]
  const uint16_t* ws;         // bf16 scales [E, N, ng]
  const int32_t* sorted_pos;  // [M*k] rows t*k+j in segment order
  const int32_t* desc;        // [E][4] (expert, segment start, rows, 0) per active slot
  const int32_t* n_active;    // [1]
  const int64_t* topk_idx;    // [M, k]
  const float* topk_w;        // [M, k]
  uint16_t* out;              // [M, N]
  int M, topk, E, N, K, G, ng;
  // nullable: the down streamer's tiled copy of the weights (k_tile_decode),
  // read in place of wp; its TPW, block and per-expert bytes
  const int32_t* wt;
  int tpw, block_bytes;
  int64_t expert_bytes;
};

// Arguments of the BF16 experts' grouped GEMMs (kernels_bf16_experts.hip).
struct Bf16ExpertArgs {
  const uint16_t* act;        // gate_up: hidden [M, K]; down: inter [M*k, K] in segment order
  const uint16_t* W;          // bf16 weights [E, N, K]
  uint16_t* out;              // gate_up: inter [M*k, I] (segment order); down: dn rows t*k+j [M*k, N]
  const int32_t* sorted_pos;  // [M*k] rows t*k+j in expert-segment order
  const int32_t* desc;        // [E][4] (expert, segment start, rows, 0) per active slot
  const int32_t* n_active;    // [1]
  int N, K, I, topk;
  int rows_total;             // M * topk routed rows (sets the row-chunk size)
};

hipError_t launch_dequant(const int32_t* packed, const uint16_t* scale, uint16_t* out,
                          int64_t rows, int K, int G, hipStream_t s);
// max_slots: upper bound of active experts (1 for dense).  self_args
// (gate_up, nullable) with self_mode (DecodeSelf): the launch works out its
// own plan and its last workgroup writes it (kSelfRoute: the routing too,
// from the router's K-split partials, TopkSortArgs with M = 1; kSelfPlan:
// from the finished top-k in idx_out); hipErrorNotSupported (nothing
// launched) where decode_self_supported or the launcher says no.
hipError_t launch_decode(int mode, DecodeArgs a, int max_slots, hipStream_t s, const TopkSortArgs* self_args = nullptr,
                         int self_mode = kSelfNone);
bool decode_self_supported(int self_mode, bool tiled, int64_t M, int64_t H, int64_t I, int64_t G, int64_t E,
                           int64_t topk);
// Tiled expert weights for the decode streamers (kernels_decode.hip): bytes
// per expert of the tiled copy of the gate_up (mode kModeGateUp) or down
// weights for group size G (0: no tiled form for H, I, G), whether that copy
// carries the group scales too, the copy, and the streamer reading it.
size_t tiled_decode_bytes_per_expert(int mode, int64_t H, int64_t I, int64_t G);
bool tiled_decode_needs_scale(int G);
hipError_t launch_tile_decode(int mode, const int32_t* packed, const uint16_t* scale, int E, int H, int I, int G,
                              int32_t* tiled, hipStream_t s);
hipError_t launch_decode_tiled(int mode, DecodeArgs a, int max_slots, hipStream_t s,
                               const TopkSortArgs* self_args = nullptr, int self_mode = kSelfNone);
// x = bf16(h + delta) -> h_out (delta may be null), y = bf16(rms_norm(x) * w)
hipError_t launch_add_rms_norm(const uint16_t* h, const uint16_t* delta, const uint16_t* w,
                               uint16_t* h_out, uint16_t* y, int64_t M, int H, float eps,
                               hipStream_t s);
hipError_t launch_combine(const uint16_t* dn, const int64_t* idx, const float* w, uint16_t* out,
                          int M, int topk, int E, int H, hipStream_t s);
// the combine (out nullable), h_out = bf16(h + out) and y = RMSNorm(h_out) * w
// in one launch (kernels_norm.hip), the bits of launch_combine followed by
// launch_add_rms_norm; topk <= 8
hipError_t launch_combine_add_rms_norm(const uint16_t* dn, const int64_t* idx, const float* tw, const uint16_t* h,
                                       const uint16_t* w, uint16_t* out, uint16_t* h_out, uint16_t* y, int64_t M,
                                       int topk, int E, int H, float eps, hipStream_t s);
// down + combine in one launch: M * topk <= kDownCombineMaxRows,
// K <= 768 and a multiple of 32; the intermediate rows in the order the
// decode gate_up writes them; the weights in the packed layout (a.wt NULL)
// or the down streamer's tiled copy (a.wt; group size 128, 32 or 64)
bool down_combine_supported(int64_t M, int64_t topk, int64_t K);
hipError_t launch_down_combine(DownCombineArgs a, hipStream_t s);
// the down streamer's tiled-copy shape for (H, I, G): TPW, block bytes and
// bytes per expert (false where there is none)
bool tiled_decode_down_geometry(int64_t H, int64_t I, int64_t G, int* tpw, int* block_bytes, int64_t* expert_bytes);
// Every plan writer's slot_rows: 0 gives one work descriptor per active
// expert; kDecodeSlotRows (the decode streamers' plans) one per 16 rows of an
// expert, so an expert with more rows than a streamer stages per pass runs as
// several slots side by side.  The descriptor array then holds up to
// plan_desc_capacity entries.
constexpr int kDecodeSlotRows = 16;
inline int64_t plan_desc_capacity(int64_t M, int64_t topk, int64_t E) {
  return E + (M * topk + kDecodeSlotRows - 1) / kDecodeSlotRows;
}

// The expert sort; with `queues` (nullable) it also zeroes the
// kPrefillQueueInts prefill work-queue counters there.  Every plan writer's
// BM is the prefill m-tile height of the tile list (a power of two), or 0 for
// plans with no tile list (counters[1] = 0): the decode streamers read none.
// slot_rows is 0 or kDecodeSlotRows.
hipError_t launch_sort(const int64_t* idx, int M, int topk, int E, int32_t* sorted_pos,
                       int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                       int BM, int slot_rows, hipStream_t s, int32_t* queues = nullptr);
// the sort over several workgroups (large batches); blockcnt holds
// sort_blocks(M * topk) * E ints
int sort_blocks(int64_t rows);
hipError_t launch_sort_multi(const int64_t* idx, int M, int topk, int E, int32_t* sorted_pos,
                             int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                             int32_t* blockcnt, int BM, int slot_rows, hipStream_t s, int32_t* queues = nullptr);
hipError_t launch_router_norm(const uint16_t* h, const uint16_t* scale, float scalar_root,
                              float eps, uint16_t* r, int M, int H, hipStream_t s);
hipError_t launch_router_logits(const uint16_t* r, const uint16_t* proj, float* partial, int M,
                                int H, int E, int ksplit, hipStream_t s);
// RMSNorm + logits partials in one launch; K split by ksplit with at most
// 12 steps of 32 per split (H <= 384 * ksplit)
hipError_t launch_router_norm_logits(const uint16_t* h, const uint16_t* scale, float scalar_root,
                                     float eps, const uint16_t* proj, float* partial, int M,
                                     int H, int E, int ksplit, hipStream_t s);
// large batches: row inverse norms into inv[M], then K-split logits partials
// [router_tok_splits(M, E)][M][E]
int router_tok_splits(int64_t M, int64_t E);
hipError_t launch_router_tok(const uint16_t* h, const uint16_t* scale, float scalar_root,
                             float eps, const uint16_t* proj, float* inv, float* partial, int M,
                             int H, int E, hipStream_t s);
// top-k and expert sort in one workgroup, M * topk <= 64, the decode router's
// kRouterMaxSplit partials
hipError_t launch_topk_sort(const float* partial, int ksplit, const uint16_t* per_expert_scale,
                            int64_t* idx, float* w, int M, int E, int topk, int32_t* sorted_pos,
                            int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                            int BM, int slot_rows, hipStream_t s);
hipError_t launch_router_topk(const float* partial, int ksplit, const uint16_t* logits_in,
                              const uint16_t* per_expert_scale, uint16_t* logits_out,
                              int64_t* idx, float* w, int M, int E, int topk, hipStream_t s);
// HybridLink pieces (kernels_hybridlink.hip): nn.LayerNorm with bf16 affine
// parameters (H % 8 == 0, H <= 8192); frag: y in the bf16 linears' fragment
// order (linear_bf16.hpp; H % 32 == 0, rows padded to a multiple of 16)
hipError_t launch_layer_norm(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                             int64_t M, int H, float eps, bool frag, hipStream_t s);
// bf16-weight linear for small batches (kernels_linear_bf16.hip), K % 32 ==
// 0, with a fused epilogue:
//   kLinGelu      out = bf16(GELU_erf(bf16(x W^T + b)))
//   kLinResidual  out = bf16(res + bf16(x W^T + b))
//   kLinGateUp    out = bf16(bf16(gelu_tanh(bf16(x W^T))) * bf16(x W2^T))
//   kLinPlain     out = bf16(x W^T)
// M rows in tiles of up to 64 (ceil(M / 64) <= 65535).
enum LinearEpilogue { kLinGelu = 0, kLinResidual = 1, kLinGateUp = 2, kLinPlain = 3 };
hipError_t launch_linear_bf16(int epi, const uint16_t* x, const uint16_t* W, const uint16_t* W2,
                              const uint16_t* bias, const uint16_t* res, uint16_t* out, int64_t M, int N,
                              int K, hipStream_t s);
// One bf16 linear (launch_linear_bf16's arguments), for the launches that run
// it beside other work.
struct LinearCall {
  int epi;
  const uint16_t *x, *W, *W2, *bias, *res;
  uint16_t* out;
  int64_t M;
  int N, K;
};
// launch_router_norm_logits with a kLinGateUp linear of at most 32 rows in the
// same launch; launch_topk_sort (one top-k round, E <= 128) with a kLinPlain
// linear of at most 16 rows.  hipErrorNotSupported (nothing launched) where
// the shapes need separate launches.
hipError_t launch_router_norm_logits_with_linear(const uint16_t* h, const uint16_t* scale, float scalar_root,
                                                 float eps, const uint16_t* proj, float* partial, int M, int H,
                                                 int E, int ksplit, const LinearCall& lin, hipStream_t s);
hipError_t launch_topk_sort_with_linear(const float* partial, int ksplit, const uint16_t* per_expert_scale,
                                        int64_t* idx, float* w, int M, int E, int topk, int32_t* sorted_pos,
                                        int32_t* offsets, int32_t* desc, int32_t* counters, int32_t* tiles,
                                        int BM, int slot_rows, const LinearCall& lin, hipStream_t s);
// FFN block row kernels (kernels_ffn.hip), one workgroup per row, H % 8 == 0,
// H <= 8192:
//   pre : h = rms(attn) * w_pa; res_out = bf16(res + h);
//         h_ff = rms(res_out) * w_pf; h2_in = rms(res_out) * w_pf2
//   post: h1 = rms(mlp) * w1; h2 = rms(moe) * w2; c = rms(bf16(h1 + h2)) * w3;
//         out = bf16(bf16(res + c) * layer_scalar)
hipError_t launch_ffn_pre(const uint16_t* attn, const uint16_t* res, const uint16_t* w_pa,
                          const uint16_t* w_pf, const uint16_t* w_pf2, uint16_t* res_out, uint16_t* h_ff,
                          uint16_t* h2_in, int64_t M, int H, float eps, hipStream_t s);
hipError_t launch_ffn_post(const uint16_t* mlp, const uint16_t* moe, const uint16_t* res,
                           const uint16_t* w1, const uint16_t* w2, const uint16_t* w3,
                           const uint16_t* layer_scalar, uint16_t* out, int64_t M, int H, float eps,
                           hipStream_t s);
// BF16 experts: grid (column tile, active slot), max_slots <= 65535
hipError_t launch_bf16_experts(int mode, Bf16ExpertArgs a, int max_slots, hipStream_t s);
// prefill grouped GEMM: one launch per stage, items = (m-tile, n-tile)
hipError_t launch_prefill(int mode, PrefillArgs a, int max_mtiles, hipStream_t s);
// the exact-form prefill GEMM (kernels_prefill_x.hip): H and I multiples of
// 64, G a power of two >= 32; items of up to kPrefillXBM rows
bool prefill_x_supported(int64_t H, int64_t I, int64_t G);
hipError_t launch_prefill_x(int mode, PrefillArgs a, int max_mtiles, hipStream_t s);
// the exact-form prefill kernel's tiled weight copy: bytes per expert of
// the gate_up (mode kModeGateUp, N = 2I, K = H) or down (N = H, K = I)
// weights, 0 where the kernel does not serve (H, I); and the copy
size_t prefill_tiled_bytes_per_expert(int mode, int64_t H, int64_t I);
hipError_t launch_tile_prefill(int mode, const int32_t* packed, int E, int H, int I, int32_t* tiled,
                               hipStream_t s);
// persistent prefill grid: the workgroups that fit at once (a multiple of the
// 8 XCDs), at most max_items
int prefill_grid_size(const void* kern, int threads, size_t lds, int max_items);

}  // namespace w4a16
