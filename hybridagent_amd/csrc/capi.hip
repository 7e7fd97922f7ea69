// C ABI of libw4a16moe.so: host-side validation, workspace carving and
// kernel launches.  See include/w4a16moe.h for the contract of each entry
// point and the reference function it replaces.
#include "w4a16moe.h"

#include "launch.hpp"
#include <algorithm>
#include <atomic>
#include <mutex>

using namespace w4a16;

namespace {

constexpr int kVersion = (0 << 16) | (2 << 8) | 0;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline bool valid_group(int64_t G) { return G >= 32 && G <= (1 << 20) && (G & (G - 1)) == 0; }

inline size_t round256(size_t b) { return (b + 255) & ~size_t(255); }

// Row-per-workgroup launches (256 threads) keep rows * 256 below 2^32.
constexpr int64_t kMaxRowLaunches = (int64_t(1) << 24) - 1;
// HybridLink: the linears' grid.y = ceil(B / 64) stays <= 65535
constexpr int64_t kMaxHybridLinkRows = int64_t(65535) * 64;

// Bump allocator over a caller-provided workspace.
struct Carve {
  char* base;
  size_t used = 0;
  explicit Carve(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
    used += round256(count * sizeof(T));
    return p;
  }
};

inline int launch_status(hipError_t e) { return e == hipSuccess ? W4A16_OK : W4A16_ERR_LAUNCH; }

// K splits of the router logits: decode sizes 16, large batches what the
// large-batch router picks for its grid
inline int router_ksplit(int64_t M, int64_t E) { return M <= 64 ? 16 : router_tok_splits(M, E); }

// Token counts up to this use the decode kernels; larger batches the
// prefill grouped-GEMM kernels.
constexpr int64_t kDecodeMaxM = 256;
// routed rows above this sort over several workgroups (two launches)
constexpr int64_t kSortMultiMinRows = 2048;
// routed rows up to this run top-k and the expert sort in one workgroup
// (measured faster than two launches up to M = 8 at top-8; slower from M = 32)
constexpr int64_t kTopkSortMaxEntries = 64;
// longest reduction the streaming kernels stage in LDS (one row per pass)
constexpr int64_t kMaxStreamK = 49152 / 2;

// Router partial logits.  `r` is workspace of M * H bf16: the normalised
// rows on the generic path, the rows' inverse norms (M floats) on the
// large-batch path.
// decode sizes with rows the fused norm + logits launch takes (the router
// partials' path below)
inline bool router_fused_norm_logits(int64_t M, int64_t H) { return M <= 64 && H <= 384 * 8; }

// The FFN block's shared MLP (backends.py:105-108): its gate/up and down
// linears, which layer_forward_impl runs inside the router's launches where
// the shapes allow.
struct SharedMlp {
  LinearCall gate_up, down;
};

// The latent harness's residual add and next norm after a layer:
// h_out = bf16(h + out), y = RMSNorm(h_out) * w (w4a16_add_rms_norm's
// arithmetic), fused into the combine launch where the layer has one.
struct AddNorm {
  const uint16_t* h;
  const uint16_t* w;
  float eps;
  uint16_t* h_out;
  uint16_t* y;
};

inline hipError_t launch_linear_call(const LinearCall& l, hipStream_t s) {
  return launch_linear_bf16(l.epi, l.x, l.W, l.W2, l.bias, l.res, l.out, l.M, l.N, l.K, s);
}

hipError_t launch_router_partials(const uint16_t* hidden, const uint16_t* scale, float root,
                                  float eps, const uint16_t* proj, uint16_t* r, float* partial,
                                  int64_t M, int64_t H, int64_t E, hipStream_t s) {
  const int ks = router_ksplit(M, E);
  // large batches: inverse norms, then logits with r formed in registers
  if (M > 64)
    return launch_router_tok(hidden, scale, root, eps, proj, reinterpret_cast<float*>(r), partial,
                             (int)M, (int)H, (int)E, s);
  // decode sizes: the norm inside the logits launch (each workgroup covers
  // all experts of 16 tokens, so it normalises its rows once)
  if (router_fused_norm_logits(M, H))
    return launch_router_norm_logits(hidden, scale, root, eps, proj, partial, (int)M, (int)H,
                                     (int)E, ks, s);
  // long rows at decode sizes: a normalisation pass into r, then the K-split
  // MFMA logits
  hipError_t e = launch_router_norm(hidden, scale, root, eps, r, (int)M, (int)H, s);
  if (e == hipSuccess) e = launch_router_logits(r, proj, partial, (int)M, (int)H, (int)E, ks, s);
  return e;
}

// One shared description of the MoE workspace so sizing and carving agree.
struct MoeLayout {
  int32_t* offsets;
  int32_t* desc;
  int32_t* counters;
  int32_t* queues;  // prefill work queues: gate_up [0, 16), down [16, 32)
  int32_t* sorted_pos;
  int32_t* tiles;
  int32_t* blockcnt;
  uint16_t* inter;
  uint16_t* dn;
  size_t bytes;
};

MoeLayout moe_layout(void* ws, int64_t M, int64_t k, int64_t E, int64_t H, int64_t I) {
  Carve c(ws);
  MoeLayout L;
  L.offsets = c.take<int32_t>(E + 1);
  L.desc = c.take<int32_t>(4 * plan_desc_capacity(M, k, E));
  L.counters = c.take<int32_t>(4);
  L.queues = c.take<int32_t>(kPrefillQueueInts);
  L.sorted_pos = c.take<int32_t>(M * k);
  L.tiles = c.take<int32_t>(M * k / kPrefillBM + E + 1);
  L.blockcnt = c.take<int32_t>(size_t(sort_blocks(M * k)) * E);
  L.inter = c.take<uint16_t>(M * k * I);
  L.dn = c.take<uint16_t>(M * k * H);
  L.bytes = c.used;
  return L;
}

// The tiled weight copies one call reads (NULL: that kernel reads the packed
// tensors), resolved from the caller's w4a16_tiled_experts.
struct Tiles {
  const int32_t* gu_decode = nullptr;
  const int32_t* dn_decode = nullptr;
  const int32_t* gu_prefill = nullptr;
  const int32_t* dn_prefill = nullptr;
};

// bytes of a tiled copy of `kind` for the shape, 0 where the kernel that
// would read it has no tiled form there
size_t tiled_need(int kind, int64_t E, int64_t H, int64_t I, int64_t G) {
  if (E <= 0 || E > kMaxExperts || H <= 0 || I <= 0 || H % 32 != 0 || I % 32 != 0 || !valid_group(G))
    return 0;
  switch (kind) {
    case W4A16_TILED_GATE_UP_DECODE:
      return (size_t)E * tiled_decode_bytes_per_expert(kModeGateUp, H, I, G);
    case W4A16_TILED_DOWN_DECODE:
      return (size_t)E * tiled_decode_bytes_per_expert(kModeDown, H, I, G);
    case W4A16_TILED_GATE_UP_PREFILL:
      return (size_t)E * prefill_tiled_bytes_per_expert(kModeGateUp, H, I);
    case W4A16_TILED_DOWN_PREFILL:
      return (size_t)E * prefill_tiled_bytes_per_expert(kModeDown, H, I);
    default:
      return 0;
  }
}

// Checks the copies against the call's shape: the tag must name the same
// expert stack (E, H, I, group size), each copy given must exist for that
// shape and hold its full size, 16-byte aligned.
int resolve_tiles(const w4a16_tiled_experts* t, int64_t E, int64_t H, int64_t I, int64_t G, Tiles* out) {
  *out = Tiles{};
  if (t == nullptr) return W4A16_OK;
  if (t->E != E || t->H != H || t->I != I || t->group_size != G) return W4A16_ERR_SHAPE;
  const struct {
    const int32_t* p;
    size_t bytes;
    int kind;
    const int32_t** dst;
  } copies[4] = {{t->gu_decode, t->gu_decode_bytes, W4A16_TILED_GATE_UP_DECODE, &out->gu_decode},
                 {t->dn_decode, t->dn_decode_bytes, W4A16_TILED_DOWN_DECODE, &out->dn_decode},
                 {t->gu_prefill, t->gu_prefill_bytes, W4A16_TILED_GATE_UP_PREFILL, &out->gu_prefill},
                 {t->dn_prefill, t->dn_prefill_bytes, W4A16_TILED_DOWN_PREFILL, &out->dn_prefill}};
  for (const auto& c : copies) {
    if (c.p == nullptr) continue;
    const size_t need = tiled_need(c.kind, E, H, I, G);
    if (need == 0) return W4A16_ERR_SHAPE;
    if (c.bytes < need) return W4A16_ERR_WORKSPACE;
    if (!aligned16(c.p)) return W4A16_ERR_ALIGN;
    *c.dst = c.p;
  }
  return W4A16_OK;
}

}  // namespace

extern "C" {

int w4a16moe_version(void) { return kVersion; }

const char* w4a16moe_status_string(int status) {
  switch (status) {
    case W4A16_OK: return "ok";
    case W4A16_ERR_NULL: return "a required pointer is NULL";
    case W4A16_ERR_SHAPE: return "a size is out of range or inconsistent";
    case W4A16_ERR_GROUP: return "unsupported group size (power of two >= 32 required)";
    case W4A16_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case W4A16_ERR_WORKSPACE: return "workspace missing or too small";
    case W4A16_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown status";
  }
}

int w4a16_dequantize(const int32_t* packed, const uint16_t* scale, uint16_t* out, int64_t rows,
                     int64_t K, int64_t group_size, void* stream) {
  if (rows < 0 || K <= 0 || K % 8 != 0 || K > (1 << 24)) return W4A16_ERR_SHAPE;
  if (!valid_group(group_size)) return W4A16_ERR_GROUP;
  if (rows == 0) return W4A16_OK;
  if (!packed || !scale || !out) return W4A16_ERR_NULL;
  if (!aligned16(out)) return W4A16_ERR_ALIGN;
  return launch_status(launch_dequant(packed, scale, out, rows, (int)K, (int)group_size,
                                      static_cast<hipStream_t>(stream)));
}

int w4a16_add_rms_norm(const uint16_t* h, const uint16_t* delta, const uint16_t* weight,
                       uint16_t* h_out, uint16_t* y, int64_t M, int64_t H, float eps,
                       void* stream) {
  // one 256-thread workgroup per row: M * 256 work-items must fit in 32 bits
  if (M < 0 || M > kMaxRowLaunches || H <= 0 || H % 8 != 0 || H > 8192) return W4A16_ERR_SHAPE;
  if (M == 0) return W4A16_OK;
  if (!h || !weight || !y || (delta && !h_out)) return W4A16_ERR_NULL;
  if (!aligned16(h) || !aligned16(weight) || !aligned16(y) || (delta && !aligned16(delta)) ||
      (h_out && !aligned16(h_out)))
    return W4A16_ERR_ALIGN;
  return launch_status(launch_add_rms_norm(h, delta, weight, h_out, y, M, (int)H, eps,
                                           static_cast<hipStream_t>(stream)));
}

// two fragment-order matrices (rows padded to 16) and one row-major
size_t w4a16_hybridlink_workspace_bytes(int64_t B, int64_t H) {
  if (B <= 0 || H <= 0) return 0;
  const size_t bp = size_t((B + 15) / 16 * 16);
  return 2 * round256(bp * H * 2) + round256(size_t(B) * H * 2);
}

int w4a16_hybridlink(const uint16_t* h, const uint16_t* ln1_w, const uint16_t* ln1_b,
                     const uint16_t* p1_w, const uint16_t* p1_b, const uint16_t* p2_w,
                     const uint16_t* p2_b, const uint16_t* ln2_w, const uint16_t* ln2_b,
                     uint16_t* out, int64_t B, int64_t H, float eps, void* workspace,
                     size_t workspace_bytes, void* stream) {
  // LayerNorm: one 256-thread workgroup per row; the linears: grid.y = ceil(B / 64) <= 65535
  if (B < 0 || B > kMaxHybridLinkRows || H <= 0 || H % 32 != 0 || H > 8192) return W4A16_ERR_SHAPE;
  if (B == 0) return W4A16_OK;
  if (!h || !ln1_w || !ln1_b || !p1_w || !p1_b || !p2_w || !p2_b || !ln2_w || !ln2_b || !out)
    return W4A16_ERR_NULL;
  if (!aligned16(h) || !aligned16(ln1_w) || !aligned16(ln1_b) || !aligned16(p1_w) ||
      !aligned16(p2_w) || !aligned16(ln2_w) || !aligned16(ln2_b) || !aligned16(out))
    return W4A16_ERR_ALIGN;
  if (workspace == nullptr || workspace_bytes < w4a16_hybridlink_workspace_bytes(B, H))
    return W4A16_ERR_WORKSPACE;
  if (!aligned16(workspace)) return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carve c(workspace);
  const int64_t Bp = (B + 15) / 16 * 16;
  uint16_t* a = c.take<uint16_t>(Bp * H);  // pre_ln(h), fragment order
  uint16_t* g = c.take<uint16_t>(Bp * H);  // GELU(proj1(...)), fragment order
  uint16_t* r = c.take<uint16_t>(B * H);   // h + proj2(...)
  hipError_t e = launch_layer_norm(h, ln1_w, ln1_b, a, B, (int)H, eps, true, s);
  if (e == hipSuccess) e = launch_linear_bf16(kLinGelu, a, p1_w, nullptr, p1_b, nullptr, g, B, (int)H, (int)H, s);
  if (e == hipSuccess) e = launch_linear_bf16(kLinResidual, g, p2_w, nullptr, p2_b, h, r, B, (int)H, (int)H, s);
  if (e == hipSuccess) e = launch_layer_norm(r, ln2_w, ln2_b, out, B, (int)H, eps, false, s);
  return launch_status(e);
}

size_t w4a16_linear_workspace_bytes(int64_t M, int64_t K, int64_t group_size) {
  (void)M;
  (void)K;
  (void)group_size;
  return 0;  // the dense path needs no scratch memory
}

int w4a16_linear(const uint16_t* x, const int32_t* w_packed, const uint16_t* w_scale,
                 const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                 int64_t group_size, void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || K % 32 != 0 || K > (1 << 24) || N > (1 << 24) ||
      M > (1 << 24))
    return W4A16_ERR_SHAPE;
  // the packed matrix is addressed by 32-bit byte offsets of one buffer descriptor
  if (N * K / 2 >= (int64_t(1) << 31)) return W4A16_ERR_SHAPE;
  if (!valid_group(group_size)) return W4A16_ERR_GROUP;
  if (M == 0) return W4A16_OK;
  if (!x || !w_packed || !w_scale || !y) return W4A16_ERR_NULL;
  if (!aligned16(x) || !aligned16(w_packed)) return W4A16_ERR_ALIGN;
  (void)workspace;
  (void)workspace_bytes;
  if (K > kMaxStreamK) return W4A16_ERR_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  DecodeArgs a{};
  a.act = x;
  a.wp = w_packed;
  a.ws = w_scale;
  a.bias = bias;
  a.out = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = (int)group_size;
  a.ng = (int)((K + group_size - 1) / group_size);
  a.topk = 1;
  a.I = 0;
  a.rows_hint = (int)(M < 16 ? M : 16);
  return launch_status(launch_decode(kModeDense, a, 1, s));
}

size_t moe_router_workspace_bytes(int64_t M, int64_t H, int64_t E) {
  if (M <= 0 || H <= 0 || E <= 0) return 0;
  return round256(size_t(M) * H * 2) + round256(size_t(router_ksplit(M, E)) * M * E * 4);
}

int moe_router_topk(const uint16_t* hidden, const uint16_t* router_scale, float scalar_root,
                    const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                    int64_t M, int64_t H, int64_t E, int64_t top_k, uint16_t* logits_out,
                    int64_t* topk_idx, float* topk_w, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (M < 0 || M > (1 << 24) || H <= 0 || H % 32 != 0 || H > (1 << 20) || E <= 0 ||
      E > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > E)
    return W4A16_ERR_SHAPE;
  if (M == 0) return W4A16_OK;
  if (!hidden || !router_scale || !proj_w || !per_expert_scale || !topk_idx || !topk_w)
    return W4A16_ERR_NULL;
  if (!aligned16(hidden) || !aligned16(proj_w) || !aligned16(router_scale)) return W4A16_ERR_ALIGN;
  const size_t need = moe_router_workspace_bytes(M, H, E);
  if (workspace == nullptr || workspace_bytes < need) return W4A16_ERR_WORKSPACE;
  if (!aligned16(workspace)) return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carve c(workspace);
  uint16_t* r = c.take<uint16_t>(M * H);
  const int ks = router_ksplit(M, E);
  float* partial = c.take<float>(size_t(ks) * M * E);
  hipError_t e = launch_router_partials(hidden, router_scale, scalar_root, eps, proj_w, r, partial,
                                        M, H, E, s);
  if (e == hipSuccess)
    e = launch_router_topk(partial, ks, nullptr, per_expert_scale, logits_out, topk_idx, topk_w,
                           (int)M, (int)E, (int)top_k, s);
  return launch_status(e);
}

int moe_topk_from_logits(const uint16_t* logits, const uint16_t* per_expert_scale, int64_t M,
                         int64_t E, int64_t top_k, int64_t* topk_idx, float* topk_w,
                         void* stream) {
  if (M < 0 || M > (1 << 24) || E <= 0 || E > kMaxExperts || top_k <= 0 || top_k > kMaxTopK ||
      top_k > E)
    return W4A16_ERR_SHAPE;
  if (M == 0) return W4A16_OK;
  if (!logits || !per_expert_scale || !topk_idx || !topk_w) return W4A16_ERR_NULL;
  return launch_status(launch_router_topk(nullptr, 0, logits, per_expert_scale, nullptr, topk_idx,
                                          topk_w, (int)M, (int)E, (int)top_k,
                                          static_cast<hipStream_t>(stream)));
}

size_t moe_sort_workspace_bytes(int64_t M, int64_t top_k, int64_t E) {
  if (M <= 0 || top_k <= 0 || E <= 0) return 0;
  return round256(size_t(E) * 16) + round256(16) + round256(size_t(M * top_k / kPrefillBM + E + 1) * 4) +
         round256(size_t(sort_blocks(M * top_k)) * E * 4);
}

int moe_sort_permute(const int64_t* topk_idx, int64_t M, int64_t top_k, int64_t E,
                     int32_t* sorted_pos, int32_t* expert_offsets, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (M < 0 || top_k <= 0 || top_k > kMaxTopK || E <= 0 || E > kMaxExperts ||
      M * top_k > (int64_t(1) << 30))
    return W4A16_ERR_SHAPE;
  if (!expert_offsets) return W4A16_ERR_NULL;
  if (M > 0 && (!topk_idx || !sorted_pos)) return W4A16_ERR_NULL;
  const size_t need = moe_sort_workspace_bytes(M > 0 ? M : 1, top_k, E);
  if (workspace == nullptr || workspace_bytes < need) return W4A16_ERR_WORKSPACE;
  Carve c(workspace);
  int32_t* desc = c.take<int32_t>(4 * E);
  int32_t* counters = c.take<int32_t>(4);
  int32_t* tiles = c.take<int32_t>(M * top_k / kPrefillBM + E + 1);
  int32_t* blockcnt = c.take<int32_t>(size_t(sort_blocks(M * top_k)) * E);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (M * top_k > kSortMultiMinRows)
    return launch_status(launch_sort_multi(topk_idx, (int)M, (int)top_k, (int)E, sorted_pos,
                                           expert_offsets, desc, counters, tiles, blockcnt,
                                           kPrefillBM, 0, s));
  return launch_status(launch_sort(topk_idx, (int)M, (int)top_k, (int)E, sorted_pos,
                                   expert_offsets, desc, counters, tiles, kPrefillBM, 0, s));
}

size_t moe_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I) {
  if (M <= 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
  return moe_layout(nullptr, M, top_k, E, H, I).bytes;
}

}  // extern "C"

namespace {

// Shared validation of the MoE entry points; fills *L on success.
int moe_check(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t G,
              void* workspace, size_t workspace_bytes, MoeLayout* L) {
  if (M < 0 || top_k <= 0 || top_k > kMaxTopK || E <= 0 || E > kMaxExperts || H <= 0 ||
      H % 32 != 0 || I <= 0 || I % 32 != 0 || H > kMaxStreamK || I > kMaxStreamK ||
      M * top_k > (int64_t(1) << 30) / (H > I ? H : I))
    return W4A16_ERR_SHAPE;
  if (!valid_group(G)) return W4A16_ERR_GROUP;
  if (M == 0) return W4A16_OK;
  const MoeLayout need = moe_layout(nullptr, M, top_k, E, H, I);
  if (workspace == nullptr || workspace_bytes < need.bytes) return W4A16_ERR_WORKSPACE;
  if (!aligned16(workspace)) return W4A16_ERR_ALIGN;
  *L = moe_layout(workspace, M, top_k, E, H, I);
  return W4A16_OK;
}

// The prefill kernels stage K in 64-wide steps and tile N by 128 weight rows
// (gate_up: 64 gate + 64 up rows); other shapes stay on the decode kernels.
inline bool use_prefill(int64_t M, int64_t H, int64_t I) {
  return M > kDecodeMaxM && H % 128 == 0 && I % 64 == 0;
}

// the exact-form prefill GEMM serves group sizes that are powers of two
// >= 32 with an even group count per row; the fallback exact-form kernel the
// rest (odd group counts, H or I below three 64-wide stages)
inline bool x_prefill(int64_t M, int64_t H, int64_t I, int64_t G) {
  return use_prefill(M, H, I) && prefill_x_supported(H, I, G);
}

// m-tile of the prefill tile list the expert sort writes
inline int plan_bm(int64_t M, int64_t H, int64_t I, int64_t G) {
  return x_prefill(M, H, I, G) ? kPrefillXBM : kPrefillBM;
}

PrefillArgs prefill_args(const MoeLayout& L, int64_t M, int64_t top_k, int64_t I, int64_t G) {
  PrefillArgs a{};
  a.sorted_pos = L.sorted_pos;
  a.offsets = L.offsets;
  a.tiles = L.tiles;
  a.counters = L.counters;
  a.topk = (int)top_k;
  a.G = (int)G;
  a.I = (int)I;
  (void)M;
  return a;
}

// most m-tiles the sort can emit: one partial tile per active expert plus
// the full ones
inline int max_mtiles(int64_t M, int64_t top_k, int64_t E, int bm = kPrefillBM) {
  const int64_t rows = M * top_k;
  return (int)(rows / bm + (rows < E ? rows : E));
}

inline int log2_int(int64_t v) {
  int r = 0;
  while ((int64_t(1) << (r + 1)) <= v) ++r;
  return r;
}

DecodeArgs expert_args(const MoeLayout& L, int64_t M, int64_t top_k, int64_t I, int64_t G) {
  DecodeArgs a{};
  a.sorted_pos = L.sorted_pos;
  a.desc = L.desc;
  a.n_active = L.counters;
  a.topk = (int)top_k;
  a.G = (int)G;
  a.I = (int)I;
  a.M = (int)M;
  // rows staged per pass: an expert usually holds at most M rows (one per
  // token); a token that routes several slots to one expert adds passes
  a.rows_hint = (int)(M < 16 ? M : 16);
  return a;
}

}  // namespace

extern "C" {

int moe_plan(const uint16_t* hidden, const int64_t* topk_idx, int64_t M, int64_t top_k,
             int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
             size_t workspace_bytes, void* stream) {
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, group_size, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!hidden || !topk_idx) return W4A16_ERR_NULL;
  if (!aligned16(hidden)) return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the decode streamers take an expert's rows as slots of kDecodeSlotRows
  // and read no m-tile list
  const bool pf = use_prefill(M, H, I);
  const int bm = pf ? plan_bm(M, H, I, group_size) : 0;
  const int sr = pf ? 0 : kDecodeSlotRows;
  hipError_t e =
      M * top_k > kSortMultiMinRows
          ? launch_sort_multi(topk_idx, (int)M, (int)top_k, (int)E, L.sorted_pos, L.offsets,
                              L.desc, L.counters, L.tiles, L.blockcnt, bm, sr, s, L.queues)
          : launch_sort(topk_idx, (int)M, (int)top_k, (int)E, L.sorted_pos, L.offsets, L.desc,
                        L.counters, L.tiles, bm, sr, s, L.queues);
  return launch_status(e);
}

}  // extern "C"

namespace {
// gate_up on either weight layout: the tiled copies in t (checked by
// resolve_tiles) serve the kernels that read them, gu_packed everything else
int gate_up_impl(const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale, const Tiles& t,
                 int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                 size_t workspace_bytes, void* stream, const TopkSortArgs* self_args = nullptr,
                 int self_mode = kSelfNone) {
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, group_size, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!hidden || !gu_packed || !gu_scale) return W4A16_ERR_NULL;
  if (!aligned16(hidden) || !aligned16(gu_packed)) return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_prefill(M, H, I, group_size)) {
    // exact form: natural hidden rows in, natural intermediate rows out
    PrefillArgs p = prefill_args(L, M, top_k, I, group_size);
    p.act = hidden;
    p.act_bytes = M * H * 2;
    p.lda = (int)H;
    p.wp = gu_packed;
    p.ws = gu_scale;
    p.out = L.inter;
    p.ldo = (int)I;
    p.N = (int)(2 * I);
    p.K = (int)H;
    p.ng = (int)((H + group_size - 1) / group_size);
    p.gshift = log2_int(group_size);
    p.rows_total = (int)(M * top_k);
    p.n_nt = (int)((I + 127) / 128);  // 128 intermediate columns per item
    p.queues = L.queues;
    p.wt = t.gu_prefill;
    return launch_status(launch_prefill_x(kModeGateUp, p, max_mtiles(M, top_k, E, kPrefillXBM), s));
  }
  if (use_prefill(M, H, I)) {
    PrefillArgs p = prefill_args(L, M, top_k, I, group_size);
    p.act = hidden;
    p.wp = gu_packed;
    p.ws = gu_scale;
    p.out = L.inter;
    p.N = (int)(2 * I);
    p.K = (int)H;
    p.ng = (int)((H + group_size - 1) / group_size);
    p.n_nt = (int)(I / 64);
    return launch_status(launch_prefill(kModeGateUp, p, max_mtiles(M, top_k, E), s));
  }
  // the plan's slots: kDecodeSlotRows rows of an expert each
  const int max_slots = (int)std::min<int64_t>(M * top_k, plan_desc_capacity(M, top_k, E));
  DecodeArgs a = expert_args(L, M, top_k, I, group_size);
  a.act = hidden;
  a.wp = gu_packed;
  a.ws = gu_scale;
  a.out = L.inter;
  a.N = (int)(2 * I);
  a.K = (int)H;
  a.ng = (int)((H + group_size - 1) / group_size);
  if (t.gu_decode != nullptr) {
    a.wp = t.gu_decode;
    return launch_status(launch_decode_tiled(kModeGateUp, a, max_slots, s, self_args, self_mode));
  }
  return launch_status(launch_decode(kModeGateUp, a, max_slots, s, self_args, self_mode));
}
}  // namespace

extern "C" {

int moe_gate_up(const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size,
                void* workspace, size_t workspace_bytes, void* stream) {
  return gate_up_impl(hidden, gu_packed, gu_scale, Tiles{}, M, top_k, E, H, I, group_size, workspace,
                      workspace_bytes, stream);
}

int moe_gate_up_tiled(const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                      const w4a16_tiled_experts* tiled, int64_t M, int64_t top_k, int64_t E, int64_t H,
                      int64_t I, int64_t group_size, void* workspace, size_t workspace_bytes, void* stream) {
  Tiles t;
  const int st = resolve_tiles(tiled, E, H, I, group_size, &t);
  if (st != W4A16_OK) return st;
  return gate_up_impl(hidden, gu_packed, gu_scale, t, M, top_k, E, H, I, group_size, workspace,
                      workspace_bytes, stream);
}

size_t w4a16_tiled_bytes(int kind, int64_t E, int64_t H, int64_t I, int64_t group_size) {
  return tiled_need(kind, E, H, I, group_size);
}

int w4a16_tile(int kind, const int32_t* packed, const uint16_t* scale, int64_t E, int64_t H, int64_t I,
               int64_t group_size, int32_t* tiled, size_t tiled_bytes, void* stream) {
  if (!valid_group(group_size)) return W4A16_ERR_GROUP;
  const size_t need = tiled_need(kind, E, H, I, group_size);
  if (need == 0) return W4A16_ERR_SHAPE;
  if (!packed || !tiled) return W4A16_ERR_NULL;
  if (!aligned16(packed) || !aligned16(tiled)) return W4A16_ERR_ALIGN;
  if (tiled_bytes < need) return W4A16_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (kind) {
    case W4A16_TILED_GATE_UP_DECODE:
    case W4A16_TILED_DOWN_DECODE:
      if (tiled_decode_needs_scale((int)group_size) && scale == nullptr) return W4A16_ERR_NULL;
      return launch_status(launch_tile_decode(kind == W4A16_TILED_GATE_UP_DECODE ? kModeGateUp : kModeDown, packed,
                                              scale, (int)E, (int)H, (int)I, (int)group_size, tiled, s));
    default:
      return launch_status(launch_tile_prefill(kind == W4A16_TILED_GATE_UP_PREFILL ? kModeGateUp : kModeDown,
                                               packed, (int)E, (int)H, (int)I, tiled, s));
  }
}

static int down_impl(const int32_t* dn_packed, const uint16_t* dn_scale, const Tiles& t, int64_t M,
                     int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                     size_t workspace_bytes, void* stream) {
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, group_size, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!dn_packed || !dn_scale) return W4A16_ERR_NULL;
  if (!aligned16(dn_packed)) return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_prefill(M, H, I, group_size)) {
    PrefillArgs p = prefill_args(L, M, top_k, I, group_size);
    p.act = L.inter;
    p.act_bytes = M * top_k * I * 2;
    p.lda = (int)I;
    p.wp = dn_packed;
    p.ws = dn_scale;
    p.out = L.dn;
    p.N = (int)H;
    p.K = (int)I;
    p.ng = (int)((I + group_size - 1) / group_size);
    p.gshift = log2_int(group_size);
    p.rows_total = (int)(M * top_k);
    p.n_nt = (int)((H + 255) / 256);  // 256 output columns per item
    p.queues = L.queues + kPrefillQueueInts / 2;
    p.wt = t.dn_prefill;
    return launch_status(launch_prefill_x(kModeDown, p, max_mtiles(M, top_k, E, kPrefillXBM), s));
  }
  if (use_prefill(M, H, I)) {
    PrefillArgs p = prefill_args(L, M, top_k, I, group_size);
    p.act = L.inter;
    p.wp = dn_packed;
    p.ws = dn_scale;
    p.out = L.dn;
    p.N = (int)H;
    p.K = (int)I;
    p.ng = (int)((I + group_size - 1) / group_size);
    p.n_nt = (int)(H / kPfBN);
    return launch_status(launch_prefill(kModeDown, p, max_mtiles(M, top_k, E), s));
  }
  // the plan's slots: kDecodeSlotRows rows of an expert each
  const int max_slots = (int)std::min<int64_t>(M * top_k, plan_desc_capacity(M, top_k, E));
  DecodeArgs a = expert_args(L, M, top_k, I, group_size);
  a.act = L.inter;
  a.wp = dn_packed;
  a.ws = dn_scale;
  a.out = L.dn;
  a.N = (int)H;
  a.K = (int)I;
  a.ng = (int)((I + group_size - 1) / group_size);
  if (t.dn_decode != nullptr) {
    a.wp = t.dn_decode;
    return launch_status(launch_decode_tiled(kModeDown, a, max_slots, s));
  }
  return launch_status(launch_decode(kModeDown, a, max_slots, s));
}

int moe_down(const int32_t* dn_packed, const uint16_t* dn_scale, int64_t M, int64_t top_k,
             int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
             size_t workspace_bytes, void* stream) {
  return down_impl(dn_packed, dn_scale, Tiles{}, M, top_k, E, H, I, group_size, workspace, workspace_bytes,
                   stream);
}

int moe_down_tiled(const int32_t* dn_packed, const uint16_t* dn_scale, const w4a16_tiled_experts* tiled, int64_t M,
                   int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                   size_t workspace_bytes, void* stream) {
  Tiles t;
  const int st = resolve_tiles(tiled, E, H, I, group_size, &t);
  if (st != W4A16_OK) return st;
  return down_impl(dn_packed, dn_scale, t, M, top_k, E, H, I, group_size, workspace, workspace_bytes, stream);
}

int moe_combine(const int64_t* topk_idx, const float* topk_w, uint16_t* out, int64_t M,
                int64_t top_k, int64_t E, int64_t H, int64_t I, void* workspace,
                size_t workspace_bytes, void* stream) {
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, 128, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!topk_idx || !topk_w || !out) return W4A16_ERR_NULL;
  if (!aligned16(out)) return W4A16_ERR_ALIGN;
  return launch_status(launch_combine(L.dn, topk_idx, topk_w, out, (int)M, (int)top_k, (int)E,
                                      (int)H, static_cast<hipStream_t>(stream)));
}

}  // extern "C"

namespace {

// Routed rows up to which the one-call forwards fuse down and combine: the
// fused launch measured faster up to 32 rows (decode layer M = 1 / 2 / 4 at
// top-8: 32.6 -> 30.0, 37.9 -> 35.0, 44.2 -> 43.0 us) and slower at 64 (M = 8:
// 59.2 -> 60.6 us), where the down streamer's 512 workgroups stream the
// weights faster than the fused kernel's 176.
constexpr int64_t kFuseDownCombineRows = 32;

// The down projection and the weighted combine of the fused forwards: at
// decode sizes with few routed rows in one launch (k_down_combine, the same
// result bit for bit), otherwise moe_down then moe_combine.
int down_and_combine(const int32_t* dn_packed, const uint16_t* dn_scale, const int64_t* topk_idx,
                     const float* topk_w, uint16_t* out, int64_t M, int64_t top_k, int64_t E,
                     int64_t H, int64_t I, int64_t group_size, void* workspace,
                     size_t workspace_bytes, void* stream, const Tiles& t, const AddNorm* an = nullptr) {
  if (use_prefill(M, H, I) || M * top_k > kFuseDownCombineRows || !down_combine_supported(M, top_k, I)) {
    int st = down_impl(dn_packed, dn_scale, t, M, top_k, E, H, I, group_size, workspace, workspace_bytes,
                       stream);
    if (st != W4A16_OK) return st;
    if (an != nullptr && top_k <= 8) {
      MoeLayout L{};
      st = moe_check(M, top_k, E, H, I, group_size, workspace, workspace_bytes, &L);
      if (st != W4A16_OK) return st;
      return launch_status(launch_combine_add_rms_norm(L.dn, topk_idx, topk_w, an->h, an->w, out, an->h_out,
                                                       an->y, M, (int)top_k, (int)E, (int)H, an->eps,
                                                       static_cast<hipStream_t>(stream)));
    }
    st = moe_combine(topk_idx, topk_w, out, M, top_k, E, H, I, workspace, workspace_bytes, stream);
    if (st == W4A16_OK && an != nullptr)
      st = launch_status(launch_add_rms_norm(an->h, out, an->w, an->h_out, an->y, M, (int)H, an->eps,
                                             static_cast<hipStream_t>(stream)));
    return st;
  }
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, group_size, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!dn_packed || !dn_scale || !topk_idx || !topk_w || !out) return W4A16_ERR_NULL;
  if (!aligned16(dn_packed) || !aligned16(out)) return W4A16_ERR_ALIGN;
  DownCombineArgs a{};
  a.act = L.inter;
  a.wp = dn_packed;
  a.ws = dn_scale;
  a.sorted_pos = L.sorted_pos;
  a.desc = L.desc;
  a.n_active = L.counters;
  a.topk_idx = topk_idx;
  a.topk_w = topk_w;
  a.out = out;
  a.M = (int)M;
  a.topk = (int)top_k;
  a.E = (int)E;
  a.N = (int)H;
  a.K = (int)I;
  a.G = (int)group_size;
  a.ng = (int)((I + group_size - 1) / group_size);
  // the down streamer's tiled copy serves the fused kernel too
  if (t.dn_decode != nullptr &&
      tiled_decode_down_geometry(H, I, group_size, &a.tpw, &a.block_bytes, &a.expert_bytes))
    a.wt = t.dn_decode;
  st = launch_status(launch_down_combine(a, static_cast<hipStream_t>(stream)));
  if (st == W4A16_OK && an != nullptr)
    st = launch_status(launch_add_rms_norm(an->h, out, an->w, an->h_out, an->y, M, (int)H, an->eps,
                                           static_cast<hipStream_t>(stream)));
  return st;
}

}  // namespace

extern "C" {

static int forward_impl(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                        const int32_t* gu_packed, const uint16_t* gu_scale, const int32_t* dn_packed,
                        const uint16_t* dn_scale, const Tiles& t, uint16_t* out, int64_t M, int64_t top_k,
                        int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                        size_t workspace_bytes, void* stream) {
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, group_size, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!hidden || !topk_idx || !topk_w || !gu_packed || !gu_scale || !dn_packed || !dn_scale ||
      !out)
    return W4A16_ERR_NULL;
  st = moe_plan(hidden, topk_idx, M, top_k, E, H, I, group_size, workspace, workspace_bytes,
                stream);
  if (st == W4A16_OK)
    st = gate_up_impl(hidden, gu_packed, gu_scale, t, M, top_k, E, H, I, group_size, workspace,
                      workspace_bytes, stream);
  if (st == W4A16_OK)
    st = down_and_combine(dn_packed, dn_scale, topk_idx, topk_w, out, M, top_k, E, H, I,
                          group_size, workspace, workspace_bytes, stream, t);
  return st;
}

int moe_forward(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                const int32_t* gu_packed, const uint16_t* gu_scale, const int32_t* dn_packed,
                const uint16_t* dn_scale, uint16_t* out, int64_t M, int64_t top_k, int64_t E,
                int64_t H, int64_t I, int64_t group_size, void* workspace,
                size_t workspace_bytes, void* stream) {
  return forward_impl(hidden, topk_idx, topk_w, gu_packed, gu_scale, dn_packed, dn_scale, Tiles{}, out, M, top_k,
                      E, H, I, group_size, workspace, workspace_bytes, stream);
}

int moe_forward_tiled(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                      const int32_t* gu_packed, const uint16_t* gu_scale, const int32_t* dn_packed,
                      const uint16_t* dn_scale, const w4a16_tiled_experts* tiled, uint16_t* out, int64_t M,
                      int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                      size_t workspace_bytes, void* stream) {
  Tiles t;
  const int st = resolve_tiles(tiled, E, H, I, group_size, &t);
  if (st != W4A16_OK) return st;
  return forward_impl(hidden, topk_idx, topk_w, gu_packed, gu_scale, dn_packed, dn_scale, t, out, M, top_k, E, H,
                      I, group_size, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// The FFN block's workspace: its row buffers, the routing, then the MoE
// layer's workspace.
struct FfnLayout {
  uint16_t* res;    // residual + rms_norm(attn_out)
  uint16_t* h_ff;   // shared-MLP input
  uint16_t* h2_in;  // experts' input
  uint16_t* inter;  // shared-MLP intermediate [M, Im]
  uint16_t* h_mlp;  // shared-MLP output
  uint16_t* moe;    // experts' output
  int64_t* idx;
  float* w;
  size_t idx_off, w_off;  // byte offsets of idx and w in the workspace
  void* moe_ws;
  size_t moe_bytes;
  size_t bytes;
};

FfnLayout ffn_layout(void* ws, int64_t M, int64_t k, int64_t E, int64_t H, int64_t I, int64_t Im) {
  Carve c(ws);
  FfnLayout L;
  L.res = c.take<uint16_t>(M * H);
  L.h_ff = c.take<uint16_t>(M * H);
  L.h2_in = c.take<uint16_t>(M * H);
  L.inter = c.take<uint16_t>(M * Im);
  L.h_mlp = c.take<uint16_t>(M * H);
  L.moe = c.take<uint16_t>(M * H);
  L.idx_off = c.used;
  L.idx = c.take<int64_t>(M * k);
  L.w_off = c.used;
  L.w = c.take<float>(M * k);
  L.moe_bytes = moe_layer_workspace_bytes(M, k, E, H, I);
  L.moe_ws = c.take<unsigned char>(L.moe_bytes);
  L.bytes = c.used;
  return L;
}

}  // namespace

extern "C" {

size_t moe_ffn_block_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                                     int64_t Im) {
  if (M <= 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0 || Im <= 0) return 0;
  return ffn_layout(nullptr, M, top_k, E, H, I, Im).bytes;
}

static int layer_forward_impl(const uint16_t* router_in, const uint16_t* router_scale, float scalar_root,
                              const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                              const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                              const int32_t* dn_packed, const uint16_t* dn_scale, const Tiles& t,
                              uint16_t* out, int64_t* topk_idx, float* topk_w, int64_t M, int64_t top_k,
                              int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                              size_t workspace_bytes, void* stream, const SharedMlp* mlp = nullptr,
                              const AddNorm* an = nullptr);

static int ffn_block_impl(const uint16_t* residual, const uint16_t* attn_out,
                          const uint16_t* post_attn_ln_w, const uint16_t* pre_ff_ln_w,
                          const uint16_t* mlp_gate_w, const uint16_t* mlp_up_w,
                          const uint16_t* mlp_down_w, const uint16_t* post_ff_ln1_w,
                          const uint16_t* router_scale, float router_scalar_root,
                          const uint16_t* router_proj_w, const uint16_t* router_per_expert_scale,
                          const uint16_t* pre_ff_ln2_w, const int32_t* gu_packed,
                          const uint16_t* gu_scale, const int32_t* dn_packed,
                          const uint16_t* dn_scale, const uint16_t* post_ff_ln2_w,
                          const uint16_t* post_ff_ln_w, const uint16_t* layer_scalar, float eps,
                          uint16_t* out, int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                          int64_t Im, int64_t group_size, void* workspace, size_t workspace_bytes,
                          void* stream, const Tiles& t) {
  // row kernels: H <= 8192, one workgroup per row; shared-MLP linears:
  // K % 32 == 0 and ceil(M / 64) <= 65535 row tiles
  if (M < 0 || M > kMaxHybridLinkRows || top_k <= 0 || top_k > E || H <= 0 || H % 32 != 0 || H > 8192 ||
      Im <= 0 || Im % 32 != 0 || Im > (1 << 16))
    return W4A16_ERR_SHAPE;
  MoeLayout none{};
  int st = moe_check(M, top_k, E, H, I, group_size, nullptr, 0, &none);
  if (st != W4A16_OK && st != W4A16_ERR_WORKSPACE) return st;
  if (M == 0) return W4A16_OK;
  if (!residual || !attn_out || !post_attn_ln_w || !pre_ff_ln_w || !mlp_gate_w || !mlp_up_w ||
      !mlp_down_w || !post_ff_ln1_w || !router_scale || !router_proj_w || !router_per_expert_scale ||
      !pre_ff_ln2_w || !gu_packed || !gu_scale || !dn_packed || !dn_scale || !post_ff_ln2_w ||
      !post_ff_ln_w || !layer_scalar || !out)
    return W4A16_ERR_NULL;
  const void* a16[] = {residual, attn_out, post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w,
                       mlp_down_w, post_ff_ln1_w, router_scale, router_proj_w, pre_ff_ln2_w,
                       gu_packed, dn_packed, post_ff_ln2_w, post_ff_ln_w, out};
  for (const void* p : a16)
    if (!aligned16(p)) return W4A16_ERR_ALIGN;
  if (workspace == nullptr || workspace_bytes < moe_ffn_block_workspace_bytes(M, top_k, E, H, I, Im))
    return W4A16_ERR_WORKSPACE;
  if (!aligned16(workspace)) return W4A16_ERR_ALIGN;
  const FfnLayout L = ffn_layout(workspace, M, top_k, E, H, I, Im);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = launch_ffn_pre(attn_out, residual, post_attn_ln_w, pre_ff_ln_w, pre_ff_ln2_w, L.res,
                                L.h_ff, L.h2_in, M, (int)H, eps, s);
  if (e != hipSuccess) return W4A16_ERR_LAUNCH;
  const SharedMlp mlp{LinearCall{kLinGateUp, L.h_ff, mlp_gate_w, mlp_up_w, nullptr, nullptr, L.inter, M, (int)Im,
                                 (int)H},
                      LinearCall{kLinPlain, L.inter, mlp_down_w, nullptr, nullptr, nullptr, L.h_mlp, M, (int)H,
                                 (int)Im}};
  st = layer_forward_impl(L.res, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale, eps,
                          L.h2_in, gu_packed, gu_scale, dn_packed, dn_scale, t, L.moe, L.idx, L.w, M, top_k, E, H,
                          I, group_size, L.moe_ws, L.moe_bytes, stream, &mlp);
  if (st != W4A16_OK) return st;
  return launch_status(launch_ffn_post(L.h_mlp, L.moe, L.res, post_ff_ln1_w, post_ff_ln2_w, post_ff_ln_w,
                                       layer_scalar, out, M, (int)H, eps, s));
}

int moe_ffn_block_forward(const uint16_t* residual, const uint16_t* attn_out,
                          const uint16_t* post_attn_ln_w, const uint16_t* pre_ff_ln_w,
                          const uint16_t* mlp_gate_w, const uint16_t* mlp_up_w,
                          const uint16_t* mlp_down_w, const uint16_t* post_ff_ln1_w,
                          const uint16_t* router_scale, float router_scalar_root,
                          const uint16_t* router_proj_w, const uint16_t* router_per_expert_scale,
                          const uint16_t* pre_ff_ln2_w, const int32_t* gu_packed,
                          const uint16_t* gu_scale, const int32_t* dn_packed,
                          const uint16_t* dn_scale, const uint16_t* post_ff_ln2_w,
                          const uint16_t* post_ff_ln_w, const uint16_t* layer_scalar, float eps,
                          uint16_t* out, int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                          int64_t Im, int64_t group_size, void* workspace, size_t workspace_bytes,
                          void* stream) {
  return ffn_block_impl(residual, attn_out, post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w,
                        post_ff_ln1_w, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale,
                        pre_ff_ln2_w, gu_packed, gu_scale, dn_packed, dn_scale, post_ff_ln2_w, post_ff_ln_w,
                        layer_scalar, eps, out, M, top_k, E, H, I, Im, group_size, workspace, workspace_bytes,
                        stream, Tiles{});
}

int moe_ffn_block_forward_tiled(const uint16_t* residual, const uint16_t* attn_out,
                                const uint16_t* post_attn_ln_w, const uint16_t* pre_ff_ln_w,
                                const uint16_t* mlp_gate_w, const uint16_t* mlp_up_w,
                                const uint16_t* mlp_down_w, const uint16_t* post_ff_ln1_w,
                                const uint16_t* router_scale, float router_scalar_root,
                                const uint16_t* router_proj_w, const uint16_t* router_per_expert_scale,
                                const uint16_t* pre_ff_ln2_w, const int32_t* gu_packed, const uint16_t* gu_scale,
                                const int32_t* dn_packed, const uint16_t* dn_scale,
                                const w4a16_tiled_experts* tiled, const uint16_t* post_ff_ln2_w,
                                const uint16_t* post_ff_ln_w, const uint16_t* layer_scalar, float eps, uint16_t* out,
                                int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t Im,
                                int64_t group_size, void* workspace, size_t workspace_bytes, void* stream) {
  Tiles t;
  const int st = resolve_tiles(tiled, E, H, I, group_size, &t);
  if (st != W4A16_OK) return st;
  return ffn_block_impl(residual, attn_out, post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w,
                        post_ff_ln1_w, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale,
                        pre_ff_ln2_w, gu_packed, gu_scale, dn_packed, dn_scale, post_ff_ln2_w, post_ff_ln_w,
                        layer_scalar, eps, out, M, top_k, E, H, I, Im, group_size, workspace, workspace_bytes,
                        stream, t);
}

int moe_ffn_block_routing_offsets(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t Im,
                                  size_t* idx_offset, size_t* w_offset) {
  if (M <= 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0 || Im <= 0) return W4A16_ERR_SHAPE;
  if (!idx_offset || !w_offset) return W4A16_ERR_NULL;
  const FfnLayout L = ffn_layout(nullptr, M, top_k, E, H, I, Im);
  *idx_offset = L.idx_off;
  *w_offset = L.w_off;
  return W4A16_OK;
}

size_t moe_bf16_experts_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I) {
  return moe_workspace_bytes(M, top_k, E, H, I);
}

int moe_bf16_experts_forward(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                             const uint16_t* gate_up_proj, const uint16_t* down_proj, uint16_t* out,
                             int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                             void* workspace, size_t workspace_bytes, void* stream) {
  // the MoE shape checks (group size unused: any valid one)
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, 128, workspace, workspace_bytes, &L);
  if (st != W4A16_OK || M == 0) return st;
  if (!hidden || !topk_idx || !topk_w || !gate_up_proj || !down_proj || !out) return W4A16_ERR_NULL;
  if (!aligned16(hidden) || !aligned16(gate_up_proj) || !aligned16(down_proj) || !aligned16(out))
    return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e =
      M * top_k > kSortMultiMinRows
          ? launch_sort_multi(topk_idx, (int)M, (int)top_k, (int)E, L.sorted_pos, L.offsets, L.desc,
                              L.counters, L.tiles, L.blockcnt, kPrefillBM, 0, s)
          : launch_sort(topk_idx, (int)M, (int)top_k, (int)E, L.sorted_pos, L.offsets, L.desc,
                        L.counters, L.tiles, kPrefillBM, 0, s);
  const int max_slots = (int)(M * top_k < E ? M * top_k : E);
  Bf16ExpertArgs a{};
  a.sorted_pos = L.sorted_pos;
  a.desc = L.desc;
  a.n_active = L.counters;
  a.I = (int)I;
  a.topk = (int)top_k;
  a.rows_total = (int)(M * top_k);
  if (e == hipSuccess) {
    a.act = hidden;
    a.W = gate_up_proj;
    a.out = L.inter;
    a.N = (int)(2 * I);
    a.K = (int)H;
    e = launch_bf16_experts(kModeGateUp, a, max_slots, s);
  }
  if (e == hipSuccess) {
    a.act = L.inter;
    a.W = down_proj;
    a.out = L.dn;
    a.N = (int)H;
    a.K = (int)I;
    e = launch_bf16_experts(kModeDown, a, max_slots, s);
  }
  if (e == hipSuccess) e = launch_combine(L.dn, topk_idx, topk_w, out, (int)M, (int)top_k, (int)E, (int)H, s);
  return launch_status(e);
}

}  // extern "C"

// moe_forward_static's scratch: one array per GPU the library runs on, held
// until the process ends.  Host code never uses this name as an address (on
// the host it is a stand-in, not device memory): static_scratch() looks up
// each device's copy once, with that device current, and every later use
// goes through the pointer it returns.
static __device__ __align__(256) unsigned char scratch[W4A16_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch` (the kernels' workspace for
// moe_forward_static); fails if the stream belongs to another device.
int static_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return W4A16_ERR_LAUNCH;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) return W4A16_ERR_LAUNCH;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
        return W4A16_ERR_LAUNCH;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return W4A16_OK;
}

}  // namespace

extern "C" {

int moe_forward_static(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                       const int32_t* gu_packed, const uint16_t* gu_scale,
                       const int32_t* dn_packed, const uint16_t* dn_scale, uint16_t* out,
                       int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                       int64_t group_size, void* stream) {
  // the shape checks of moe_forward (with no workspace, valid shapes report
  // W4A16_ERR_WORKSPACE), then the scratch limit
  MoeLayout none{};
  int st = moe_check(M, top_k, E, H, I, group_size, nullptr, 0, &none);
  if (st != W4A16_OK && st != W4A16_ERR_WORKSPACE) return st;
  if (M == 0) return W4A16_OK;
  if (moe_workspace_bytes(M, top_k, E, H, I) > W4A16_STATIC_SCRATCH_BYTES) return W4A16_ERR_SHAPE;
  if (!hidden || !topk_idx || !topk_w || !gu_packed || !gu_scale || !dn_packed || !dn_scale ||
      !out)
    return W4A16_ERR_NULL;
  void* ws = nullptr;
  st = static_scratch(static_cast<hipStream_t>(stream), &ws);
  if (st != W4A16_OK) return st;
  return moe_forward(hidden, topk_idx, topk_w, gu_packed, gu_scale, dn_packed, dn_scale, out, M,
                     top_k, E, H, I, group_size, ws, W4A16_STATIC_SCRATCH_BYTES, stream);
}

size_t moe_layer_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I) {
  if (M <= 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
  return moe_layout(nullptr, M, top_k, E, H, I).bytes + moe_router_workspace_bytes(M, H, E);
}

static int layer_forward_impl(const uint16_t* router_in, const uint16_t* router_scale, float scalar_root,
                              const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                              const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                              const int32_t* dn_packed, const uint16_t* dn_scale, const Tiles& t,
                              uint16_t* out, int64_t* topk_idx, float* topk_w, int64_t M, int64_t top_k,
                              int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                              size_t workspace_bytes, void* stream, const SharedMlp* mlp, const AddNorm* an) {
  if (M < 0 || M > (1 << 24) || top_k > E) return W4A16_ERR_SHAPE;
  if (M == 0) {
    MoeLayout dummy{};
    return moe_check(0, top_k, E, H, I, group_size, nullptr, 0, &dummy);
  }
  if (workspace == nullptr || workspace_bytes < moe_layer_workspace_bytes(M, top_k, E, H, I))
    return W4A16_ERR_WORKSPACE;
  const size_t moe_bytes = moe_layout(nullptr, M, top_k, E, H, I).bytes;
  MoeLayout L{};
  int st = moe_check(M, top_k, E, H, I, group_size, workspace, moe_bytes, &L);
  if (st != W4A16_OK) return st;
  if (!router_in || !router_scale || !proj_w || !per_expert_scale || !hidden || !gu_packed ||
      !gu_scale || !dn_packed || !dn_scale || !out || !topk_idx || !topk_w)
    return W4A16_ERR_NULL;
  if (!aligned16(router_in) || !aligned16(proj_w) || !aligned16(router_scale) || !aligned16(hidden) ||
      !aligned16(gu_packed) || !aligned16(dn_packed) || !aligned16(out))
    return W4A16_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carve c(static_cast<char*>(workspace) + moe_bytes);
  uint16_t* r = c.take<uint16_t>(M * H);
  float* partial = c.take<float>(size_t(router_ksplit(M, E)) * M * E);
  // the shared MLP's linears (FFN block) ride in the router's launches where
  // the shapes allow, else they run as launches of their own
  bool mlp_gu = mlp == nullptr, mlp_dn = mlp == nullptr;
  hipError_t e = hipErrorNotSupported;
  if (!mlp_gu && router_fused_norm_logits(M, H))
    e = launch_router_norm_logits_with_linear(router_in, router_scale, scalar_root, eps, proj_w, partial, (int)M,
                                              (int)H, (int)E, router_ksplit(M, E), mlp->gate_up, s);
  if (e == hipSuccess) {
    mlp_gu = true;
  } else {
    if (e != hipErrorNotSupported) return W4A16_ERR_LAUNCH;
    e = mlp_gu ? hipSuccess : launch_linear_call(mlp->gate_up, s);
    mlp_gu = true;
    if (e == hipSuccess)
      e = launch_router_partials(router_in, router_scale, scalar_root, eps, proj_w, r, partial, M, H, E, s);
    if (e != hipSuccess) return W4A16_ERR_LAUNCH;
  }
  // one token (and no shared MLP to place): the gate_up launch routes too --
  // its last workgroup runs the top-k + sort, which writes the routing and
  // the plan the down stage reads, and every other workgroup finds its
  // expert from the router partials itself -- one launch fewer on the chain
  if (mlp == nullptr && decode_self_supported(kSelfRoute, t.gu_decode != nullptr, M, H, I, group_size, E, top_k)) {
    const TopkSortArgs ta{partial, per_expert_scale, topk_idx, topk_w, 1, (int)E, (int)top_k,
                          L.sorted_pos, L.offsets, L.desc, L.counters, L.tiles, 0, kDecodeSlotRows};
    st = gate_up_impl(hidden, gu_packed, gu_scale, t, M, top_k, E, H, I, group_size, workspace, moe_bytes, stream,
                      &ta, kSelfRoute);
    if (st == W4A16_OK)
      st = down_and_combine(dn_packed, dn_scale, topk_idx, topk_w, out, M, top_k, E, H, I, group_size, workspace,
                            moe_bytes, stream, t, an);
    return st;
  }
  if (M * top_k <= kTopkSortMaxEntries) {
    // small batches: top-k and the expert sort in one workgroup
    e = hipErrorNotSupported;
    if (!mlp_dn)
      e = launch_topk_sort_with_linear(partial, router_ksplit(M, E), per_expert_scale, topk_idx, topk_w, (int)M,
                                       (int)E, (int)top_k, L.sorted_pos, L.offsets, L.desc, L.counters, L.tiles,
                                       0, kDecodeSlotRows, mlp->down, s);
    if (e == hipSuccess) {
      mlp_dn = true;
    } else {
      if (e != hipErrorNotSupported) return W4A16_ERR_LAUNCH;
      e = launch_topk_sort(partial, router_ksplit(M, E), per_expert_scale, topk_idx, topk_w, (int)M,
                           (int)E, (int)top_k, L.sorted_pos, L.offsets, L.desc, L.counters, L.tiles,
                           0, kDecodeSlotRows, s);
      if (e != hipSuccess) return W4A16_ERR_LAUNCH;
    }
  } else {
    e = launch_router_topk(partial, router_ksplit(M, E), nullptr, per_expert_scale, nullptr, topk_idx,
                           topk_w, (int)M, (int)E, (int)top_k, s);
    if (e != hipSuccess) return W4A16_ERR_LAUNCH;
    if (!mlp_dn && launch_linear_call(mlp->down, s) != hipSuccess) return W4A16_ERR_LAUNCH;
    mlp_dn = true;
    // decode sizes: the gate_up launch sorts the finished top-k itself (its
    // last workgroup writes the plan the down stage reads) -- no sort launch
    if (!use_prefill(M, H, I) &&
        decode_self_supported(kSelfPlan, t.gu_decode != nullptr, M, H, I, group_size, E, top_k)) {
      const TopkSortArgs ta{nullptr, nullptr, topk_idx, nullptr, (int)M, (int)E, (int)top_k,
                            L.sorted_pos, L.offsets, L.desc, L.counters, L.tiles, 0, kDecodeSlotRows};
      // (a shape the launcher runs narrow is refused before any launch and
      // takes the sort launch below)
      st = gate_up_impl(hidden, gu_packed, gu_scale, t, M, top_k, E, H, I, group_size, workspace, moe_bytes, stream,
                        &ta, kSelfPlan);
      if (st == W4A16_OK)
        return down_and_combine(dn_packed, dn_scale, topk_idx, topk_w, out, M, top_k, E, H, I, group_size,
                                workspace, moe_bytes, stream, t, an);
    }
    st = moe_plan(hidden, topk_idx, M, top_k, E, H, I, group_size, workspace, moe_bytes, stream);
    if (st != W4A16_OK) return st;
  }
  if (!mlp_dn && launch_linear_call(mlp->down, s) != hipSuccess) return W4A16_ERR_LAUNCH;
  st = gate_up_impl(hidden, gu_packed, gu_scale, t, M, top_k, E, H, I, group_size, workspace,
                    moe_bytes, stream);
  if (st == W4A16_OK)
    st = down_and_combine(dn_packed, dn_scale, topk_idx, topk_w, out, M, top_k, E, H, I,
                          group_size, workspace, moe_bytes, stream, t, an);
  return st;
}

int moe_layer_forward(const uint16_t* router_in, const uint16_t* router_scale, float scalar_root,
                      const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                      const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                      const int32_t* dn_packed, const uint16_t* dn_scale, uint16_t* out,
                      int64_t* topk_idx, float* topk_w, int64_t M, int64_t top_k, int64_t E,
                      int64_t H, int64_t I, int64_t group_size, void* workspace,
                      size_t workspace_bytes, void* stream) {
  return layer_forward_impl(router_in, router_scale, scalar_root, proj_w, per_expert_scale, eps, hidden, gu_packed,
                            gu_scale, dn_packed, dn_scale, Tiles{}, out, topk_idx, topk_w, M, top_k, E, H, I,
                            group_size, workspace, workspace_bytes, stream);
}

int moe_layer_forward_tiled(const uint16_t* router_in, const uint16_t* router_scale, float scalar_root,
                            const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                            const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                            const int32_t* dn_packed, const uint16_t* dn_scale, const w4a16_tiled_experts* tiled,
                            uint16_t* out, int64_t* topk_idx, float* topk_w, int64_t M, int64_t top_k, int64_t E,
                            int64_t H, int64_t I, int64_t group_size, void* workspace, size_t workspace_bytes,
                            void* stream) {
  Tiles t;
  const int st = resolve_tiles(tiled, E, H, I, group_size, &t);
  if (st != W4A16_OK) return st;
  return layer_forward_impl(router_in, router_scale, scalar_root, proj_w, per_expert_scale, eps, hidden, gu_packed,
                            gu_scale, dn_packed, dn_scale, t, out, topk_idx, topk_w, M, top_k, E, H, I, group_size,
                            workspace, workspace_bytes, stream);
}

int moe_layer_forward_add_norm(const uint16_t* router_in, const uint16_t* router_scale, float scalar_root,
                               const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                               const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                               const int32_t* dn_packed, const uint16_t* dn_scale,
                               const w4a16_tiled_experts* tiled, uint16_t* out, int64_t* topk_idx, float* topk_w,
                               const uint16_t* norm_w, float norm_eps, uint16_t* h_out, uint16_t* y_out, int64_t M,
                               int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                               size_t workspace_bytes, void* stream) {
  // the norm kernels hold a row in one 256-thread workgroup: H <= 8192
  if (H > 8192) return W4A16_ERR_SHAPE;
  if (M > 0 && (!norm_w || !h_out || !y_out)) return W4A16_ERR_NULL;
  if (M > 0 && (!aligned16(norm_w) || !aligned16(h_out) || !aligned16(y_out))) return W4A16_ERR_ALIGN;
  Tiles t;
  if (tiled != nullptr) {
    const int st = resolve_tiles(tiled, E, H, I, group_size, &t);
    if (st != W4A16_OK) return st;
  }
  const AddNorm an{router_in, norm_w, norm_eps, h_out, y_out};
  return layer_forward_impl(router_in, router_scale, scalar_root, proj_w, per_expert_scale, eps, hidden, gu_packed,
                            gu_scale, dn_packed, dn_scale, t, out, topk_idx, topk_w, M, top_k, E, H, I, group_size,
                            workspace, workspace_bytes, stream, nullptr, &an);
}

}  // extern "C"
