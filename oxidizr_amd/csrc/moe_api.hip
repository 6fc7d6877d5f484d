// C ABI of the MoE layer: plan, buffer layouts and the forward / backward
// launch sequences.  Declared in include/moe_hip.h.
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/moe_hip.h"
#include "kernels.hpp"

using namespace moe;

namespace {

thread_local std::string g_last_error;

moe_status fail(moe_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

#define HIP_TRY(expr)                                                                   \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      return fail(_e == hipErrorOutOfMemory ? MOE_ERR_OOM : MOE_ERR_HIP, "%s: %s (%s:%d)", \
                  #expr, hipGetErrorString(_e), __FILE__, __LINE__);                    \
  } while (0)

#define LAUNCH_CHECK()                                                                   \
  do {                                                                                   \
    hipError_t _e = hipGetLastError();                                                   \
    if (_e != hipSuccess)                                                                \
      return fail(MOE_ERR_HIP, "kernel launch: %s (%s:%d)", hipGetErrorString(_e), __FILE__, \
                  __LINE__);                                                             \
  } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Bump allocator over a caller buffer: records offsets of named regions.
struct Carve {
  size_t off = 0;
  size_t take(size_t bytes) {
    size_t o = off;
    off = align_up(off + bytes);
    return o;
  }
};

struct SavedLayout {
  size_t f[MOE_SAVED_NUM_FIELDS];
  size_t fbytes[MOE_SAVED_NUM_FIELDS];
  size_t tile_prefix, sG, sU, sA;
  size_t sGbytes, sUbytes, sAbytes;
  size_t total;
};

// A named region of the workspace: phase 0 regions are the forward's scratch
// (they never overlap each other), phase 1 the backward's (likewise); the two
// phases alias, since a call runs one or the other.
struct WsSpan {
  const char* name;
  size_t off, bytes;
  int phase;
};
constexpr int kMaxWsSpans = 40;

struct WsLayout {
  // forward
  size_t block_hist, block_base, colpart, ghist, gbase, gpart, rpart, sY, infer;
  // backward
  size_t dw, dwp, dY, dG, dU, dXp, dlogits, dlogits_t, sdG, sdU, dxs, splitk_router, splitk_shared,
      recomp, dxm, dwn, dwn_a, dwn_b, xorder;
  size_t total;
  size_t fwd_total;  // bytes a forward-only call touches (the forward regions)
  WsSpan span[kMaxWsSpans];
  int nspan = 0;
};

int elt_size(int dtype) { return dtype == MOE_DTYPE_F32 ? 4 : 2; }

// The fused router kernel (router GEMM + routing + the 16-token groups'
// histograms and probability sums) applies to plans (bf16 or fp32) with up to
// kFusedRouterMaxExperts experts and more than kRouteSmallTokens tokens (the
// small-token path keeps k_router_small, whose 16 x 16 blocks spread a few
// tokens over more workgroups).  With more experts a workgroup that owns every
// expert of its tokens re-reads the whole router weight per 16 tokens; there
// the tiled router GEMM and k_route stay separate.  fp32 (config 1: T = 1024,
// H = 384, E = 8): router, route and dispatch stages 19 + 8 + 15 us fused,
// against 31 + 14 + 22 us as the tiled GEMM (8 workgroups), k_route, k_hist,
// k_scan and k_scatter (step 0.357 -> 0.322 ms).
bool fused_router(const moe_config& c, int64_t T) {
  return (c.dtype == MOE_DTYPE_BF16 || c.dtype == MOE_DTYPE_F32) &&
         c.num_experts <= kFusedRouterMaxExperts && T > kRouteSmallTokens;
}
// Chunks of H the tiled router GEMM splits its k-loop into (k_router_logits_split):
// one per 1792 columns from H = 3584 up (config 5: 7168 -> 4 chunks of 28
// k-tiles), so its T / 128 x E / 128 tiles fill the CUs.  Depends on H only.
int router_splits(const moe_config& c) {
  return c.hidden >= 3584 ? std::min(8, c.hidden / 1792) : 1;
}
// Which router GEMM a forward over T tokens runs.  The router GEMM has N = E:
// up to kRouterSmallMaxExperts experts the 16 x 16 blocks of k_router_small
// fill the GPU better than 128 x 128 tiles (config 2, E = 16: 31 -> 12 us; at
// E = 64 the tiles are faster).
constexpr int kRouterSmallMaxExperts = 32;
enum class RouterPath { Fused, Small, Split, Tiled };
RouterPath router_path(const moe_config& c, int64_t T) {
  if (fused_router(c, T)) return RouterPath::Fused;
  if (c.dtype == MOE_DTYPE_BF16 && (T <= kSkinnyMaxTokens || c.num_experts <= kRouterSmallMaxExperts))
    return RouterPath::Small;
  return router_splits(c) > 1 ? RouterPath::Split : RouterPath::Tiled;
}
// The split router GEMM's partials are summed and routed by k_reduce_route
// (routing of one 16-token group per workgroup) for up to this many experts.
constexpr int kReduceRouteMaxExperts = 256;
// Whether the router path also routes the tokens and writes the 16-token
// groups' histograms and probability sums (the fused router, or the split
// router GEMM with k_reduce_route): the dispatch then scans those groups and
// the gather writes the permutation.  Always T > kRouteSmallTokens.
bool group_routing(const moe_config& c, int64_t T) {
  const RouterPath rp = router_path(c, T);
  return rp == RouterPath::Fused || (rp == RouterPath::Split && T > kRouteSmallTokens &&
                                     c.num_experts <= kReduceRouteMaxExperts);
}
template <class C>
int router_kchunk(const moe_config& c) {
  const int n = router_splits(c);
  return ((c.hidden + n - 1) / n + C::BK - 1) / C::BK * C::BK;
}

// Buffer loads take 32-bit byte offsets and kOobOffset (2^31) must lie beyond
// every resource: no operand extent may reach this many bytes.
constexpr int64_t kMaxExtentBytes = int64_t(1) << 31;
int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
int round8(int v) { return (v + 7) / 8 * 8; }

// Launch sizes that the workspace regions are planned for; the launches and
// moe_workspace_check both take them from here.
// Blocks of k_hist / k_scatter (256 tokens each).
int hist_blocks(int64_t T) { return ceil_div(T, 256); }
// 16-token groups of the fused router (its histograms, bases and sums).
int route_groups(int64_t T) { return ceil_div(T, 16); }
// Row blocks of the mean-probability column sums: 64 tokens each, or 64 of
// the fused router's 16-token groups.
int colsum_rows(int64_t T, bool routed) {
  return routed ? ceil_div(route_groups(T), 64) : ceil_div(T, 64);
}
// Levels of the RMSNorm weight gradient's 16-ary reduction tree over nrow
// partial rows: level(R, G, which) reduces R rows to G into buffer `which`
// (0, 1, 0, ...); the last <= 16 rows are reduced into the output.
template <class F>
void norm_tree(int nrow, F&& level) {
  int R = nrow, which = 0;
  while (R > 16) {
    const int G = ceil_div(R, 16);
    level(R, G, which);
    which ^= 1;
    R = G;
  }
}

// Split of a dense (all-token) weight gradient over K = tokens into fixed
// chunks (each at least four k-tiles).  The count minimises a cost model in
// units of one workgroup k-tile: rounds of workgroups on 256 CUs times k-tiles
// per chunk, plus, when split, the fp32 partial tiles written and read back by
// k_splitk_reduce (8 bytes per output element and chunk at ~5 TB/s, against
// ~3.9 TFLOP/s of MFMA work per CU: 3.1 * M * N / (BM * BN * BK) units per
// chunk).  The split depends only on the shapes, never on timing.
struct SplitPlan {
  int nsplit, kchunk;
};
template <class C>
SplitPlan plan_split(int M, int N, int K) {
  if (K <= 0) return {1, C::BK};  // no tokens: nothing to split
  const int tiles = ceil_div(M, C::BM) * ceil_div(N, C::BN);
  const int nkt = ceil_div(K, C::BK);
  const int most = K / (4 * C::BK) > 1 ? K / (4 * C::BK) : 1;
  const double red = 3.1 * (double)M * N / ((double)C::BM * C::BN * C::BK);
  int best = 1;
  double best_cost = 0;
  for (int ns = 1; ns <= most && ns <= 64; ++ns) {
    const double cost = (double)ceil_div((int64_t)tiles * ns, 256) * ceil_div(nkt, ns) +
                        (ns > 1 ? red * ns : 0.0);
    if (ns == 1 || cost < best_cost) {
      best = ns;
      best_cost = cost;
    }
  }
  const int chunk = ceil_div(ceil_div(K, best), C::BK) * C::BK;
  return {ceil_div(K, chunk), chunk};
}

// fp32 partial-tile bytes of one dense weight gradient (NA outputs of M x N
// over T tokens) as launch_dense_wgrad splits it: 0 when it runs unsplit.
template <typename D, int NA>
size_t dense_wgrad_partial_bytes(int M, int N, int T) {
  const SplitPlan sp = plan_split<WgradTiling<D, NA>>(M, N, T);
  return sp.nsplit > 1 ? (size_t)NA * sp.nsplit * (size_t)M * N * 4 : 0;
}

// fp32 partial-tile bytes of the largest dense weight gradient of one backward:
// the router's, or the shared expert's (they run concurrently, on separate
// buffers).  Planned with the tilings the launches use (WgradTiling), so the
// split counts agree; launch_dense_wgrad also refuses a split that would not
// fit.
template <typename D>
size_t splitk_bytes(const moe_config& c, int64_t T, bool shared) {
  const int H = c.hidden, E = c.num_experts, S = c.shared_intermediate;
  if (!shared) return dense_wgrad_partial_bytes<D, 1>(E, H, (int)T);
  if (S == 0) return 0;
  return std::max(dense_wgrad_partial_bytes<D, 1>(H, S, (int)T),
                  dense_wgrad_partial_bytes<D, 2>(S, H, (int)T));
}

}  // namespace

// Scratch of moe_forward_noalloc: a static device array standing in for the
// caller's workspace (one copy per GPU, held until the process ends).  Host
// code never passes the array's name to a kernel: its device address, per
// device, comes from hipGetSymbolAddress at plan creation (resolve_scratch).
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

struct moe_plan {
  moe_config cfg;
  int device;
  // workgroups of a persistent grouped weight-gradient launch: one per CU
  // (its tilings hold one workgroup per CU), rounded down to whole XCD rounds
  int wgrad_slots = 256;
  void* scratch_ptr = nullptr;  // device address of `scratch` on this plan's device
  // device pointer tables: 0 gate, 1 up, 2 down (weights); 3..5 their grads
  void** d_tab = nullptr;
  // Pinned host staging for table uploads: a ring of kTabSlots slots of 6 E
  // pointers.  A slot is refilled only after the copy that last read it has
  // run (its event), so an upload never waits for the stream as a whole.
  static constexpr int kTabSlots = 16;
  void** h_tab = nullptr;
  // The gate/up weight gradient's whole-experts-per-XCD flag of the last
  // backward, read back without waiting (pinned copy + event): when it was
  // set, the next backward launches only the persistent blocks (no blocks
  // that would only exit).  A stale or unknown flag changes the grid, never
  // the results.
  int* h_xflag = nullptr;
  hipEvent_t xflag_ev = nullptr;
  bool xflag_pending = false;
  int xflag = 0;
  hipEvent_t tab_ev[kTabSlots] = {};
  bool tab_ev_pending[kTabSlots] = {};
  int tab_next = 0;
  std::vector<const void*> cached[6];
  uint32_t profile_mask = 0;   // stages timed with HIP events (bit per moe_stage)
  struct Pending { int stage; hipEvent_t a, b; };
  std::vector<Pending> pending;
  std::vector<hipEvent_t> free_events;
  float stage_ms[MOE_NUM_STAGES] = {};
  int32_t stage_calls[MOE_NUM_STAGES] = {};
  // The shared expert does not depend on routing: it runs on a second stream
  // (default priority), forked from and joined back into the caller's stream
  // within each call, and fills the routed GEMMs' partial rounds of work.
  hipStream_t aux = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  hipEvent_t sdx = nullptr;  // backward: the shared expert's input gradient is ready
  // The backward's routed weight gradients need only dY / dG / dU and the
  // routing state: they run on a third stream, beside the input-gradient
  // GEMMs and the router backward on the call's stream.
  // In the forward the same stream sums the mean router probabilities (needed
  // only by the losses) while the call's stream dispatches.
  hipStream_t wgs = nullptr;
  hipEvent_t wfork = nullptr, wmid = nullptr, wjoin = nullptr;
  int overlap = 1;  // 0: serial; 1: shared-expert and weight-gradient streams; 2: shared only
  hipStream_t shared_stream(hipStream_t s) const { return overlap && aux ? aux : s; }
  hipStream_t wgrad_stream(hipStream_t s) const { return overlap == 1 && wgs ? wgs : s; }

  int E() const { return cfg.num_experts; }
  int es() const { return elt_size(cfg.dtype); }

  // Which state a layout holds.  All: routing and every activation (the
  // default `saved`, and the activations a recomputing backward rebuilds);
  // Transient: the state of a forward that no backward reads (no gate / up
  // pre-activations); Routing: the routing state alone (the `saved` of a plan
  // with recompute_activations).
  enum class Keep { All, Transient, Routing };
  SavedLayout saved_layout(int64_t T, Keep keep) const {
    const int E = cfg.num_experts, k = cfg.experts_per_tok, H = cfg.hidden,
              I = cfg.intermediate, S = cfg.shared_intermediate;
    const int64_t TK = T * k;
    const size_t b = es();
    SavedLayout L{};
    Carve c;
    auto fld = [&](int id, size_t bytes) { L.f[id] = c.take(bytes); L.fbytes[id] = bytes; };
    fld(MOE_SAVED_LOGITS, 4 * T * E);
    fld(MOE_SAVED_PROBS, 4 * T * E);
    fld(MOE_SAVED_LSE, 4 * T);
    fld(MOE_SAVED_TOPK_IDX, 4 * TK);
    fld(MOE_SAVED_TOPK_W, 4 * TK);
    fld(MOE_SAVED_COUNTS, 4 * (size_t)E);
    fld(MOE_SAVED_OFFSETS, 4 * (size_t)(E + 1));
    fld(MOE_SAVED_PERM, 4 * TK);
    fld(MOE_SAVED_INV_PERM, 4 * TK);
    fld(MOE_SAVED_MEAN_PROB, 4 * (size_t)E);
    L.tile_prefix = c.take(4 * (size_t)kTilePrefixes * kNumTileBM * (E + 1));
    const bool act = keep != Keep::Routing, pre = keep == Keep::All;
    // the GEMMs read x through the permutation: no permuted copy is kept
    fld(MOE_SAVED_X_PERM, 0);
    fld(MOE_SAVED_GATE_ACT, pre ? b * TK * I : 0);
    fld(MOE_SAVED_UP_ACT, pre ? b * TK * I : 0);
    fld(MOE_SAVED_SWIGLU, act ? b * TK * I : 0);
    // the expert outputs feed the forward's combine only (the backward forms
    // the combine weights' gradient from d_out Wd and A): transient state
    fld(MOE_SAVED_EXPERT_OUT, keep == Keep::Transient ? b * TK * H : 0);
    const bool blk = cfg.fused_block != 0 && act;
    fld(MOE_SAVED_RSTD, blk ? 4 * (size_t)T : 0);
    fld(MOE_SAVED_NORM_X, blk ? b * T * H : 0);
    L.sGbytes = L.sUbytes = pre ? b * T * S : 0;
    L.sAbytes = act ? b * T * S : 0;
    L.sG = c.take(L.sGbytes);
    L.sU = c.take(L.sUbytes);
    L.sA = c.take(L.sAbytes);
    L.total = c.off;
    return L;
  }

  // layout of the caller's `saved` buffer
  SavedLayout kept_layout(int64_t T) const {
    return saved_layout(T, cfg.recompute_activations ? Keep::Routing : Keep::All);
  }

  WsLayout ws_layout(int64_t T) const {
    const int E = cfg.num_experts, k = cfg.experts_per_tok, H = cfg.hidden,
              I = cfg.intermediate, S = cfg.shared_intermediate;
    const int64_t TK = T * k;
    const size_t b = es();
    const int nb = hist_blocks(T), nrb = colsum_rows(T, false);
    WsLayout L{};
    Carve f, g;
    auto put = [&](Carve& c, const char* name, size_t bytes) {
      const size_t o = c.take(bytes);
      if (L.nspan < kMaxWsSpans) L.span[L.nspan++] = {name, o, bytes, &c == &f ? 0 : 1};
      return o;
    };
    L.block_hist = put(f, "block_hist", 4 * (size_t)nb * E);
    L.block_base = put(f, "block_base", 4 * (size_t)nb * E);
    L.colpart = put(f, "colpart", 4 * (size_t)nrb * E);
    // fused router: per 16-token group histograms, dispatch bases and
    // probability column sums
    const size_t ng = group_routing(cfg, T) ? (size_t)route_groups(T) * E : 0;
    L.ghist = put(f, "ghist", 4 * ng);
    L.gbase = put(f, "gbase", 4 * ng);
    L.gpart = put(f, "gpart", 4 * ng);
    // split router GEMM: fp32 partial logits per chunk of H
    const int rs = router_path(cfg, T) == RouterPath::Split ? router_splits(cfg) : 1;
    L.rpart = put(f, "rpart", rs > 1 ? 4 * (size_t)rs * T * E : 0);
    L.sY = put(f, "sY", b * T * H);
    // forward-only calls keep their routing and activations here, clear of
    // the forward scratch above (the backward regions below are unused then)
    L.infer = put(f, "infer", saved_layout(T, Keep::Transient).total);
    // column partials of the router-bias gradient (offset 0)
    put(g, "bias_colpart", 4 * (size_t)nrb * E);
    L.dw = put(g, "dw", 4 * TK);
    // the combine weights' gradient per 32-column block of the down
    // projection's input gradient
    L.dwp = put(g, "dwp", 4 * (size_t)ceil_div(I, 32) * TK);
    // the weighted d_out rows of the down projection's weight gradient, then
    // (same stream, after it) the weighted token rows of the gate/up one
    L.dY = put(g, "dY", b * TK * H);
    L.dG = put(g, "dG", b * TK * I);
    L.dU = put(g, "dU", b * TK * I);
    L.dXp = put(g, "dXp", b * TK * H);
    L.dlogits = put(g, "dlogits", 4 * T * E);
    L.dlogits_t = put(g, "dlogits_t", b * T * round8(E));
    L.sdG = put(g, "sdG", b * T * S);
    L.sdU = put(g, "sdU", b * T * S);
    L.dxs = put(g, "dxs", b * T * H);
    const bool f32 = cfg.dtype == MOE_DTYPE_F32;
    L.splitk_router = put(g, "splitk_router", f32 ? splitk_bytes<float>(cfg, T, false)
                                                  : splitk_bytes<bf16_t>(cfg, T, false));
    L.splitk_shared = put(g, "splitk_shared", f32 ? splitk_bytes<float>(cfg, T, true)
                                                  : splitk_bytes<bf16_t>(cfg, T, true));
    // a recomputing backward rebuilds every activation here first
    L.recomp = put(g, "recomp", cfg.recompute_activations ? saved_layout(T, Keep::All).total : 0);
    // fused block: the layer's input gradient, then the RMSNorm weight
    // gradient's partial rows and two levels of their fixed-order reduction
    const bool blk = cfg.fused_block != 0;
    const int nrow = ceil_div(T, kRmsRows);
    L.dxm = put(g, "dxm", blk ? b * T * H : 0);
    L.dwn = put(g, "dwn", blk ? 4 * (size_t)nrow * H : 0);
    L.dwn_a = put(g, "dwn_a", blk ? 4 * (size_t)ceil_div(nrow, 16) * H : 0);
    L.dwn_b = put(g, "dwn_b", blk ? 4 * (size_t)ceil_div(nrow, 256) * H : 0);
    // expert order of the gate/up weight gradient over the 8 XCDs and its flag
    L.xorder = put(g, "xorder", 4 * (size_t)(E + 1));

    L.total = f.off > g.off ? f.off : g.off;
    L.fwd_total = f.off;
    return L;
  }

  hipEvent_t event() {
    if (!free_events.empty()) {
      hipEvent_t e = free_events.back();
      free_events.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};

namespace {

// Records events around one stage when profiling is on.
struct StageTimer {
  moe_plan* p;
  hipStream_t s;
  int stage;
  hipEvent_t a = nullptr;
  StageTimer(moe_plan* p_, hipStream_t s_, int st) : p(p_), s(s_), stage(st) {
    if ((p->profile_mask >> st) & 1u) {
      a = p->event();
      if (a) (void)hipEventRecord(a, s);
    }
  }
  ~StageTimer() {
    if (a) {
      hipEvent_t b = p->event();
      if (b) {
        (void)hipEventRecord(b, s);
        p->pending.push_back({stage, a, b});
      } else {
        p->free_events.push_back(a);
      }
    }
  }
};

// Work forked from the call's stream s onto a side stream of the plan is
// joined back with `ev`: join() records ev on the side stream and makes s wait
// for it.  A fork that is not joined explicitly (an error return in between)
// is joined when the guard goes out of scope, so no side-stream work is ever
// left unordered with the caller's stream.
struct SideJoin {
  hipStream_t s = nullptr, side = nullptr;
  hipEvent_t ev = nullptr;
  bool armed = false;
  // fork: side waits for everything enqueued on s so far (fork_ev)
  hipError_t fork(hipStream_t s_, hipStream_t side_, hipEvent_t fork_ev, hipEvent_t join_ev) {
    s = s_;
    side = side_;
    ev = join_ev;
    if (side == s) return hipSuccess;
    hipError_t e = hipEventRecord(fork_ev, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(side, fork_ev, 0);
    armed = e == hipSuccess;
    return e;
  }
  hipError_t join() {
    if (!armed) return hipSuccess;
    armed = false;
    hipError_t e = hipEventRecord(ev, side);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, ev, 0);
    return e;
  }
  ~SideJoin() { (void)join(); }
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Copies the three host pointer tables tabs[0..2] into device tables
// first..first + 2 when any of them changed since the last upload.  Every
// pointer is checked before any state changes, so a refused call leaves the
// cache and the device tables as they were.  The copy reads a pinned staging
// slot of the ring; the host waits only for the copy that last used that slot
// (kTabSlots uploads earlier), never for the stream.
moe_status upload_tables(moe_plan* p, hipStream_t s, int first, const void* const* tabs[3]) {
  const int E = p->E();
  bool changed = false;
  for (int i = 0; i < 3; ++i) {
    if (!tabs[i]) return fail(MOE_ERR_INVALID, "pointer table %d is NULL", first + i);
    auto& c = p->cached[first + i];
    if (c.size() != (size_t)E || memcmp(c.data(), tabs[i], sizeof(void*) * E) != 0) changed = true;
  }
  if (!changed) return MOE_OK;
  for (int i = 0; i < 3; ++i)
    for (int e = 0; e < E; ++e)
      if (!tabs[i][e] || !aligned16(tabs[i][e]))
        return fail(MOE_ERR_INVALID, "expert %d pointer %d is NULL or not 16-byte aligned", e,
                    first + i);
  // Under graph capture the copy below would be recorded as a node that
  // replays whatever the staging slot holds later (the ring reuses it), and
  // waiting for the slot's event is not allowed there: a capture must find
  // the tables already on the device.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(MOE_ERR_UNSUPPORTED,
                "the expert pointer tables changed while the stream is capturing a graph; call "
                "once with the same tables before capture");
  const int slot = p->tab_next;
  if (p->tab_ev_pending[slot]) {
    HIP_TRY(hipEventSynchronize(p->tab_ev[slot]));
    p->tab_ev_pending[slot] = false;
  }
  void** h = p->h_tab + (size_t)slot * 6 * E + (size_t)first * E;
  for (int i = 0; i < 3; ++i) memcpy(h + (size_t)i * E, tabs[i], sizeof(void*) * E);
  HIP_TRY(hipMemcpyAsync(p->d_tab + (size_t)first * E, h, sizeof(void*) * 3 * E,
                         hipMemcpyHostToDevice, s));
  HIP_TRY(hipEventRecord(p->tab_ev[slot], s));
  p->tab_ev_pending[slot] = true;
  p->tab_next = (slot + 1) % moe_plan::kTabSlots;
  for (int i = 0; i < 3; ++i) p->cached[first + i].assign(tabs[i], tabs[i] + E);
  return MOE_OK;
}

// Clears n bytes of device memory at q on stream s with a kernel (graph
// capture records no memset node for it).
moe_status zero_async(hipStream_t s, void* q, size_t n) {
  if (!q || n == 0) return MOE_OK;
  const int64_t vecs = ((int64_t)n + 15) / 16;
  hipLaunchKernelGGL(k_zero, dim3((unsigned)((vecs + 255) / 256)), dim3(256), 0, s, (uint8_t*)q,
                     (int64_t)n);
  LAUNCH_CHECK();
  return MOE_OK;
}

int route_epl(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16; }

template <int EPL>
void launch_route(hipStream_t s, int grid, const float* logits, int T, int E, int k, float tau,
                  int norm, float* probs, float* lse, int* idx, float* w) {
  hipLaunchKernelGGL((k_route<EPL>), dim3(grid), dim3(256), 0, s, logits, T, E, k, tau, norm,
                     probs, lse, idx, w);
}

// Routing (from logits already in saved), losses' P statistics and dispatch.
// pjoin != null: the mean probabilities P may be summed on the plan's
// weight-gradient stream, forked through *pjoin; the caller joins it before
// reading P.

template <int NEB, typename D>
void launch_router_route(hipStream_t s, int T, const D* x, const D* wr, const float* b,
                         int H, int E, int k, float tau, int norm, float* logits, float* probs,
                         float* lse, int* idx, float* w, int* ghist, float* gpart) {
  hipLaunchKernelGGL((k_router_route<D, NEB>), dim3(route_groups(T)), dim3(64 * kRouterWaves), 0, s,
                     x, wr, b, T, H, E, k, tau, norm, logits, probs, lse, idx, w, ghist, gpart);
}

// Routing (from logits already in saved, unless `routed`: the fused router
// kernel has written the routing decisions too), losses' P statistics and
// dispatch.  With `routed` (T > kRouteSmallTokens) the dispatch stops after
// k_scan: the caller writes perm and inv_perm (k_scatter_groups from the
// group bases at W.gbase).
template <typename D>
moe_status run_routing(moe_plan* p, hipStream_t s, int64_t T64, char* saved, char* ws,
                       const SavedLayout& L, const WsLayout& W, SideJoin* pjoin,
                       bool routed = false) {
  const moe_config& c = p->cfg;
  const int T = (int)T64, E = c.num_experts, k = c.experts_per_tok;
  float* logits = (float*)(saved + L.f[MOE_SAVED_LOGITS]);
  float* probs = (float*)(saved + L.f[MOE_SAVED_PROBS]);
  float* lse = (float*)(saved + L.f[MOE_SAVED_LSE]);
  int* idx = (int*)(saved + L.f[MOE_SAVED_TOPK_IDX]);
  float* w = (float*)(saved + L.f[MOE_SAVED_TOPK_W]);
  int* counts = (int*)(saved + L.f[MOE_SAVED_COUNTS]);
  int* offsets = (int*)(saved + L.f[MOE_SAVED_OFFSETS]);
  int* perm = (int*)(saved + L.f[MOE_SAVED_PERM]);
  int* inv = (int*)(saved + L.f[MOE_SAVED_INV_PERM]);
  float* P = (float*)(saved + L.f[MOE_SAVED_MEAN_PROB]);
  int* tprefix = (int*)(saved + L.tile_prefix);
  {
    StageTimer st(p, s, MOE_STAGE_ROUTE);
    const int grid = ceil_div(T, 4);
    const float tau = c.router_temperature;
    if (!routed) switch (route_epl(E)) {
      case 1: launch_route<1>(s, grid, logits, T, E, k, tau, c.norm_topk_prob, probs, lse, idx, w); break;
      case 2: launch_route<2>(s, grid, logits, T, E, k, tau, c.norm_topk_prob, probs, lse, idx, w); break;
      case 4: launch_route<4>(s, grid, logits, T, E, k, tau, c.norm_topk_prob, probs, lse, idx, w); break;
      case 8: launch_route<8>(s, grid, logits, T, E, k, tau, c.norm_topk_prob, probs, lse, idx, w); break;
      default: launch_route<16>(s, grid, logits, T, E, k, tau, c.norm_topk_prob, probs, lse, idx, w); break;
    }
    LAUNCH_CHECK();
    if (T <= kRouteSmallTokens) {  // P and the whole dispatch in one workgroup
      hipLaunchKernelGGL(k_dispatch_small, dim3(1), dim3(1024), 0, s, idx, probs, T, E, k,
                         1.0f / (float)T, P, counts, offsets, tprefix, perm, inv);
      LAUNCH_CHECK();
      return MOE_OK;
    }
    const hipStream_t ps = pjoin ? p->wgrad_stream(s) : s;
    if (pjoin) HIP_TRY(pjoin->fork(s, ps, p->wfork, p->wjoin));
    if (routed) {  // P from the fused router's per-group sums, in two fixed-order levels
      const int ng = route_groups(T), nrb = colsum_rows(T, true);
      float* part = (float*)(ws + W.colpart);
      hipLaunchKernelGGL(k_colsum_partial, dim3(ceil_div(E, 64), nrb), dim3(256), 0, ps,
                         (const float*)(ws + W.gpart), ng, E, part);
      hipLaunchKernelGGL(k_colsum_final, dim3(ceil_div(E, 256)), dim3(256), 0, ps, part, nrb, E,
                         1.0f / (float)T, P);
    } else {
      const int nrb = colsum_rows(T, false);
      float* part = (float*)(ws + W.colpart);
      hipLaunchKernelGGL(k_colsum_partial, dim3(ceil_div(E, 64), nrb), dim3(256), 0, ps, probs,
                         T, E, part);
      hipLaunchKernelGGL(k_colsum_final, dim3(ceil_div(E, 256)), dim3(256), 0, ps, part, nrb, E,
                         1.0f / (float)T, P);
    }
    LAUNCH_CHECK();
  }
  {
    StageTimer st(p, s, MOE_STAGE_DISPATCH);
    if (routed) {  // the fused router counted its 16-token groups' choices
      const int ng = route_groups(T);
      int* gb = (int*)(ws + W.gbase);
      hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, s, (const int*)(ws + W.ghist), ng, E, gb,
                         counts, offsets, tprefix);
    } else {
      const int nb = hist_blocks(T);
      int* bh = (int*)(ws + W.block_hist);
      int* bb = (int*)(ws + W.block_base);
      hipLaunchKernelGGL(k_hist, dim3(nb), dim3(256), sizeof(int) * E, s, idx, T, k, E, bh);
      hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, s, bh, nb, E, bb, counts, offsets, tprefix);
      hipLaunchKernelGGL(k_scatter, dim3(nb), dim3(256), sizeof(int) * 16 * E, s, idx, T, k, E,
                         bb, perm, inv);
    }
    LAUNCH_CHECK();
  }
  return MOE_OK;
}

// Index of a row-tile height in kTileBM (the row-grouped tilings use 128
// (fp32) and 256 (bf16) rows).
constexpr int tile_slot(int bm) { return bm == kF32RowTile ? 0 : bm == 256 ? 1 : 2; }
static_assert(kNumTileBM == 3, "tile_slot covers the heights of kTileBM");

// Blocks of a K-grouped (weight-gradient) launch over `groups` groups or
// split chunks of an M x N output: each takes 8 * ceil(tiles / 8) blocks.
inline int kgrouped_grid(int groups, int M, int N, int BM, int BN) {
  return groups * 8 * ceil_div(ceil_div(M, BM) * ceil_div(N, BN), 8);
}

// Weight gradient of a dense (all-token) GEMM: out_x[m, n] = alpha * sum_t
// P_x[t, m] Q[t, n], split over tokens when that fills the GPU better.  The
// fp32 partials of a split must fit the partial_bytes of `partial` (else an
// error, before anything is launched).
template <typename D, int NA>
moe_status launch_dense_wgrad(hipStream_t s, const D* P0, const D* P1, int64_t ldp, const D* Q,
                              int64_t ldq, int T, int M, int N, float alpha, D* o0, D* o1,
                              float* partial, size_t partial_bytes) {
  using C = WgradTiling<D, NA>;
  const SplitPlan sp = plan_split<C>(M, N, T);
  if (sp.nsplit > 1) {
    const size_t need = dense_wgrad_partial_bytes<D, NA>(M, N, T);
    if (need > partial_bytes)
      return fail(MOE_ERR_UNSUPPORTED,
                  "weight-gradient split of %d chunks needs %zu bytes of partials, the workspace "
                  "holds %zu",
                  sp.nsplit, need, partial_bytes);
  }
  const KGroups kg{nullptr, 1, T, sp.nsplit, sp.kchunk, 1, nullptr};
  const int grid = kgrouped_grid(sp.nsplit, M, N, C::BM, C::BN);
  hipLaunchKernelGGL((k_wgrad<D, NA, false>), dim3(grid), dim3(C::THREADS), 0, s, P0, P1, ldp, Q,
                     ldq, kg, M, N, alpha, nullptr, o0, nullptr, o1, partial, grid, 0);
  if (sp.nsplit > 1) {
    const int64_t MN = (int64_t)M * N;
    hipLaunchKernelGGL(k_splitk_reduce<D>, dim3(ceil_div(MN, 2048), NA), dim3(256), 0, s, partial,
                       sp.nsplit, MN, alpha, o0, o1);
  }
  LAUNCH_CHECK();
  return MOE_OK;
}

// Pointers to the routing state and the activations of one call.  The
// routing state lives in `saved` (or, for a forward-only call, the
// workspace); the activations live in `saved` unless the plan recomputes
// them (forward: transient workspace region; backward: rebuilt in the
// workspace before use).  G, U, sG, sU are null where they are not kept.
template <typename D>
struct State {
  float *logits, *probs, *lse, *w, *P;
  int *idx, *counts, *offsets, *perm, *inv, *tprefix;
  D *G, *U, *A, *Y, *sG, *sU, *sA;
  State(char* rb, const SavedLayout& LR, char* ab, const SavedLayout& LA) {
    auto r = [&](int f) { return rb + LR.f[f]; };
    auto a = [&](int f) { return LA.fbytes[f] ? (D*)(ab + LA.f[f]) : nullptr; };
    logits = (float*)r(MOE_SAVED_LOGITS);
    probs = (float*)r(MOE_SAVED_PROBS);
    lse = (float*)r(MOE_SAVED_LSE);
    idx = (int*)r(MOE_SAVED_TOPK_IDX);
    w = (float*)r(MOE_SAVED_TOPK_W);
    counts = (int*)r(MOE_SAVED_COUNTS);
    offsets = (int*)r(MOE_SAVED_OFFSETS);
    perm = (int*)r(MOE_SAVED_PERM);
    inv = (int*)r(MOE_SAVED_INV_PERM);
    P = (float*)r(MOE_SAVED_MEAN_PROB);
    tprefix = (int*)(rb + LR.tile_prefix);
    G = a(MOE_SAVED_GATE_ACT);
    U = a(MOE_SAVED_UP_ACT);
    A = a(MOE_SAVED_SWIGLU);
    Y = a(MOE_SAVED_EXPERT_OUT);
    sG = LA.sGbytes ? (D*)(ab + LA.sG) : nullptr;
    sU = LA.sUbytes ? (D*)(ab + LA.sU) : nullptr;
    sA = LA.sAbytes ? (D*)(ab + LA.sA) : nullptr;
  }
};

// Shared expert forward over all T tokens on stream ss: G, U (when kept), A,
// and the down projection into sY when sY is not null.
// Calls f(tiling, grid) for a dense (shared-expert) launch of tiling C over
// T rows and N columns: C, or its 384-row tiles when those fill fewer whole
// rounds of 256 CUs, a 384-row tile counted at kDense384Cost tenths of a
// 256-row one (a k-tile brings 25 % more operand rows for 50 % more MFMA
// work).  The last row tile runs as the shortest tiling that covers it.
constexpr int kDense384Cost = 14;
template <typename D, class C, class F>
void with_dense_tiling(int T, int N, F&& f) {
  const int64_t nN = ceil_div(N, C::BN);
  if constexpr (has_half_rows<D, C>()) {
    using C3 = Rows384<C>;
    const int64_t r256 = ceil_div(ceil_div(T, C::BM) * nN, (int64_t)256);
    const int64_t r384 = ceil_div(ceil_div(T, C3::AR) * nN, (int64_t)256);
    if (kDense384Cost * r384 < 10 * r256) {
      f(C3{}, (int)(ceil_div(T, C3::AR) * nN));
      return;
    }
  }
  f(C{}, (int)(ceil_div(T, C::BM) * nN));
}

template <typename D>
void shared_fwd(moe_plan* p, hipStream_t ss, int T, const D* x, const moe_weights* w, D* sG,
                D* sU, D* sA, D* sY) {
  using CG = typename Tilings<D>::GateUp;
  using CB = typename Tilings<D>::Big;
  const int H = p->cfg.hidden, S = p->cfg.shared_intermediate;
  const bool skinny = std::is_same<D, bf16_t>::value && T <= kSkinnyMaxTokens;
  if (skinny && T <= 16) {
    hipLaunchKernelGGL((k_skinny_fwd<true, false>), dim3(ceil_div(S, kSkinnyRows)), dim3(256), kSkinnyLdsReserve, ss,
                       (const bf16_t*)x, nullptr, 1, 0, nullptr, 1, T, nullptr, (const bf16_t*)w->shared_gate,
                       nullptr, (const bf16_t*)w->shared_up, H, S, (bf16_t*)sG, (bf16_t*)sU,
                       (bf16_t*)sA);
    if (sY)
      hipLaunchKernelGGL((k_skinny_fwd<false, false>), dim3(ceil_div(H, kSkinnyRows)), dim3(256), kSkinnyLdsReserve, ss,
                         (const bf16_t*)sA, nullptr, 1, 0, nullptr, 1, T, nullptr, (const bf16_t*)w->shared_down,
                         nullptr, nullptr, S, H, (bf16_t*)sY, nullptr, nullptr);
  } else if (skinny) {
    hipLaunchKernelGGL((k_skinny_fwd<true, true>), dim3(ceil_div(S, kSkinnyRows)), dim3(256), 0, ss,
                       (const bf16_t*)x, nullptr, 1, 0, nullptr, 1, T, nullptr, (const bf16_t*)w->shared_gate,
                       nullptr, (const bf16_t*)w->shared_up, H, S, (bf16_t*)sG, (bf16_t*)sU,
                       (bf16_t*)sA);
    if (sY)
      hipLaunchKernelGGL((k_skinny_fwd<false, true>), dim3(ceil_div(H, kSkinnyRows)), dim3(256), 0, ss,
                         (const bf16_t*)sA, nullptr, 1, 0, nullptr, 1, T, nullptr, (const bf16_t*)w->shared_down,
                         nullptr, nullptr, S, H, (bf16_t*)sY, nullptr, nullptr);
  } else {
    const RowGroups dense{nullptr, nullptr, nullptr, nullptr, 1, T, 0, 0};
    with_dense_tiling<D, CG>(T, S, [&](auto c, int grid) {
      using C = decltype(c);
      hipLaunchKernelGGL((k_gateup_fwd<D, false, C>), dim3(grid), dim3(C::THREADS), 0, ss, x, dense,
                         nullptr, (const D*)w->shared_gate, nullptr, (const D*)w->shared_up, H, S,
                         sG, sU, sA, nullptr, 0, 1);
    });
    if (sY)
      with_dense_tiling<D, CB>(T, H, [&](auto c, int grid) {
        using C = decltype(c);
        hipLaunchKernelGGL((k_down_fwd<D, false, C>), dim3(grid), dim3(C::THREADS), 0, ss, sA, dense,
                           nullptr, (const D*)w->shared_down, S, H, sY, nullptr);
      });
  }
}

// Rounds of 384-row tiles over the CUs a row-grouped launch must hold to take
// them: with fewer, the launch's last partial round costs more than the taller
// tiles save.
constexpr int kRows384Rounds = 4;

// Calls f(tiling, row groups, grid(N)) for a row-grouped launch of tiling C
// with N output columns: the tile prefixes of C::BM, and a grid
// of the row-tile upper bound TK / BM + E times the column tiles, rounded up
// to whole rounds of the 8 XCDs (xcd_slot2).  Half tiles run last when they
// have a half-height tiling and the groups average at least two row tiles:
// with fewer rows per expert (config 5: 256) the weight panels dominate the
// traffic, and a half tile that runs apart from its expert's big tiles reads
// them again (measured: config 2 gate/up forward 296 -> 249 us, config 5
// row-grouped GEMMs 3-4 % slower).
template <typename D, class C, bool ROWS384 = true, class F>
void with_row_tiling(const int* offsets, const int* tprefix_all, int E, int64_t TK, F&& f) {
  if constexpr (ROWS384 && has_half_rows<D, C>()) {
    // 384-row tiles, the half tiles (at most 192 rows) after the big ones,
    // when the groups average at least two of them and the launch holds at
    // least four rounds of them over 256 CUs at six column tiles (I = 1408):
    // config 3 gate/up forward 1.22 -> 1.11 ms, gate/up input gradient 1.25 ->
    // 1.22 ms, down forward 0.566 -> 0.55 ms; config 2 (16384 rows) would fill
    // fewer rounds (its routed GEMMs 8-17 % slower).  The down projection's
    // input gradient keeps 256-row tiles (ROWS384 = false: config 3 0.86 ->
    // 0.89 ms with them).
    using C3 = Rows384<C>;
    if (TK >= 2 * (int64_t)C3::AR * E && 6 * TK >= (int64_t)kRows384Rounds * 256 * C3::AR) {
      const int* tp = tprefix_all + kTilePrefixes * tile_slot(C3::AR) * (E + 1);
      const int mt = ceil_div(TK, C3::AR) + E;
      static_assert(tall_rows_for(C3::AR) == 0, "384-row tiles take no tails");
      f(C3{}, RowGroups{offsets, tp, tp + (E + 1), tp + 2 * (E + 1), E, (int)TK, 1, 0},
        [mt](int N) { return 8 * ceil_div(mt * ceil_div(N, C3::BN), 8); });
      return;
    }
  }
  const int* tp = tprefix_all + kTilePrefixes * tile_slot(C::BM) * (E + 1);
  const int mt = ceil_div(TK, C::BM) + E;
  const int half_last = has_half_rows<D, C>() && TK >= 2 * (int64_t)C::BM * E;
  // the prefixes (k_scan) merge short tails into tall tiles exactly where the
  // kernels' row tilings have them
  static_assert(tall_rows_for(C::BM) == (has_half_rows<D, C>() ? C::BM / 4 : 0), "tall tiles");
  f(C{}, RowGroups{offsets, tp, tp + (E + 1), tp + 2 * (E + 1), E, (int)TK, half_last,
                   tall_rows_for(C::BM)},
    [mt](int N) { return 8 * ceil_div(mt * ceil_div(N, C::BN), 8); });
}

// Routed experts forward on stream s: G, U (when kept), A and the
// per-assignment expert outputs Y (when st.Y is set: a recomputing backward
// needs none).  The GEMMs read each assignment's token row of x through the
// permutation (no permuted copy of x).  `timed`: record the stages.
// `gbase` (not null): the dispatch stopped after k_scan over the fused
// router's 16-token groups, whose bases gbase holds; k_scatter_groups
// then writes perm and inv_perm.
template <typename D>
moe_status routed_fwd(moe_plan* p, hipStream_t s, int T, const D* x, const State<D>& st,
                      bool timed, const int* gbase = nullptr) {
  using CG = typename Tilings<D>::GateUp;
  using CB = typename Tilings<D>::Big;
  const moe_config& c = p->cfg;
  const int H = c.hidden, E = c.num_experts, k = c.experts_per_tok, I = c.intermediate;
  const int64_t TK = (int64_t)T * k;
  auto stage = [&](int id) { return timed ? id : MOE_STAGE_RECOMPUTE; };
  // few tokens: no expert holds more than T rows, stream the weights instead
  const bool skinny = std::is_same<D, bf16_t>::value && T <= kSkinnyMaxTokens;
  if (gbase) {  // the dispatch's last launch
    StageTimer tm(p, s, stage(MOE_STAGE_DISPATCH));
    hipLaunchKernelGGL(k_scatter_groups, dim3(ceil_div(T, 4)), dim3(256), 0, s, st.idx, T, k, E,
                       gbase, st.perm, st.inv);
    LAUNCH_CHECK();
  }
  const bf16_t* xsrc = (const bf16_t*)x;
  const int* xrow = st.perm;
  const D* const* tg = (const D* const*)p->d_tab;
  const D* const* tu = (const D* const*)(p->d_tab + E);
  const D* const* td = (const D* const*)(p->d_tab + 2 * E);
  {
    StageTimer tm(p, s, stage(MOE_STAGE_GATEUP_FWD));
    if (skinny) {
      hipLaunchKernelGGL((k_skinny_fwd<true, false>), dim3(E * ceil_div(I, kSkinnyRows)), dim3(256), kSkinnyLdsReserve, s,
                         xsrc, xrow, k, T, st.offsets, E, 0, (const bf16_t* const*)tg, nullptr,
                         (const bf16_t* const*)tu, nullptr, H, I, (bf16_t*)st.G, (bf16_t*)st.U,
                         (bf16_t*)st.A);
      if (T > 16)
        hipLaunchKernelGGL((k_skinny_fwd<true, true>), dim3(max_wide_groups(TK, E) * ceil_div(I, kSkinnyRows)), dim3(256), 0, s,
                           xsrc, xrow, k, T, st.offsets, E, 0, (const bf16_t* const*)tg,
                           nullptr, (const bf16_t* const*)tu, nullptr, H, I, (bf16_t*)st.G,
                           (bf16_t*)st.U, (bf16_t*)st.A);
    } else {
      with_row_tiling<D, CG>(st.offsets, st.tprefix, E, TK, [&](auto c, const RowGroups& r, auto grid) {
        using C = decltype(c);
        hipLaunchKernelGGL((k_gateup_fwd<D, true, C>), dim3(grid(I)), dim3(C::THREADS), 0,
                           s, x, r, tg, nullptr, tu, nullptr, H, I, st.G, st.U, st.A, st.perm,
                           T, k);
      });
    }
    LAUNCH_CHECK();
  }
  if (!st.Y) return MOE_OK;  // a recomputing backward needs no expert outputs
  {
    StageTimer tm(p, s, stage(MOE_STAGE_DOWN_FWD));
    if (skinny) {
      hipLaunchKernelGGL((k_skinny_fwd<false, false>), dim3(E * ceil_div(H, kSkinnyRows)), dim3(256), kSkinnyLdsReserve, s,
                         (const bf16_t*)st.A, nullptr, 1, 0, st.offsets, E, 0, (const bf16_t* const*)td, nullptr,
                         nullptr, nullptr, I, H, (bf16_t*)st.Y, nullptr, nullptr);
      if (T > 16)
        hipLaunchKernelGGL((k_skinny_fwd<false, true>), dim3(max_wide_groups(TK, E) * ceil_div(H, kSkinnyRows)), dim3(256), 0,
                           s, (const bf16_t*)st.A, nullptr, 1, 0, st.offsets, E, 0, (const bf16_t* const*)td,
                           nullptr, nullptr, nullptr, I, H, (bf16_t*)st.Y, nullptr, nullptr);
    } else {
      with_row_tiling<D, CB>(st.offsets, st.tprefix, E, TK, [&](auto c, const RowGroups& r, auto grid) {
        using C = decltype(c);
        hipLaunchKernelGGL((k_down_fwd<D, true, C>), dim3(grid(H)), dim3(C::THREADS), 0, s,
                           st.A, r, td, nullptr, I, H, st.Y, st.perm);
      });
    }
    LAUNCH_CHECK();
  }
  return MOE_OK;
}

template <typename D>
moe_status forward_impl(moe_plan* p, hipStream_t s, int64_t T64, const D* x,
                        const moe_weights* w, D* out, float* aux, float* z, char* saved,
                        char* ws, const D* resid) {
  using CR = typename Tilings<D>::Router;
  using CG = typename Tilings<D>::GateUp;
  using CB = typename Tilings<D>::Big;
  static_assert(CG::BM == CB::BM, "row-grouped GEMMs share one tile-prefix table");
  const moe_config& c = p->cfg;
  const int T = (int)T64, H = c.hidden, E = c.num_experts, k = c.experts_per_tok,
            S = c.shared_intermediate;
  using Keep = moe_plan::Keep;
  // saved == nullptr: forward only (no backward follows): the state lives in
  // the workspace and the gate / up pre-activations are not written.  A plan
  // with recompute_activations keeps only the routing state in `saved`; the
  // activations of this call are transient, in the same workspace region.
  const bool train = saved != nullptr;
  const bool keep_act = train && !c.recompute_activations;
  const WsLayout W = p->ws_layout(T64);
  const SavedLayout LT = p->saved_layout(T64, Keep::Transient);
  const SavedLayout LR = train ? p->kept_layout(T64) : LT;
  char* rb = train ? saved : ws + W.infer;
  char* ab = keep_act ? saved : ws + W.infer;
  State<D> st(rb, LR, ab, keep_act ? LR : LT);
  // a kept training forward still needs the expert outputs for its combine:
  // they go to the forward-only region, unused by such a call
  if (!st.Y) st.Y = (D*)(ws + W.infer + LT.f[MOE_SAVED_EXPERT_OUT]);
  // Shared expert first, on the plan's second stream: it only needs x.
  D* sY = nullptr;
  SideJoin shared_join, p_join;
  if (S > 0) {
    const hipStream_t ss = p->shared_stream(s);
    HIP_TRY(shared_join.fork(s, ss, p->fork, p->join));
    StageTimer tm(p, ss, MOE_STAGE_SHARED_FWD);
    sY = (D*)(ws + W.sY);
    shared_fwd<D>(p, ss, T, x, w, st.sG, st.sU, st.sA, sY);
    LAUNCH_CHECK();
  }
  const bool fused = group_routing(c, T64);
  {
    StageTimer tm(p, s, MOE_STAGE_ROUTER_GEMM);
    const RouterPath rp = router_path(c, T64);
    if (rp == RouterPath::Fused) {  // router GEMM, softmax, lse and top-k in one launch
      const D* xb = x;
      const D* wrb = (const D*)w->router;
      const float* rbias = c.has_router_bias ? w->router_bias : nullptr;
      const float tau = c.router_temperature;
      const int nt = c.norm_topk_prob;
      int* gh = (int*)(ws + W.ghist);
      float* gp = (float*)(ws + W.gpart);
      if (E <= 16)
        launch_router_route<1, D>(s, T, xb, wrb, rbias, H, E, k, tau, nt, st.logits, st.probs, st.lse, st.idx, st.w, gh, gp);
      else if (E <= 32)
        launch_router_route<2, D>(s, T, xb, wrb, rbias, H, E, k, tau, nt, st.logits, st.probs, st.lse, st.idx, st.w, gh, gp);
      else
        launch_router_route<4, D>(s, T, xb, wrb, rbias, H, E, k, tau, nt, st.logits, st.probs, st.lse, st.idx, st.w, gh, gp);
    } else if (rp == RouterPath::Small) {
      hipLaunchKernelGGL(k_router_small, dim3(ceil_div(E, 16) * ceil_div(T, 16)),
                         dim3(64 * kRouterWaves), 0, s, (const bf16_t*)x,
                         (const bf16_t*)w->router, c.has_router_bias ? w->router_bias : nullptr,
                         st.logits, T, H, E);
    } else if (rp == RouterPath::Split) {
      const int ns = router_splits(c);
      float* part = (float*)(ws + W.rpart);
      const int tiles = ceil_div(T, CR::BM) * ceil_div(E, CR::BN);
      hipLaunchKernelGGL((k_router_logits_split<D, CR>), dim3(tiles * ns), dim3(CR::THREADS), 0, s,
                         x, (const D*)w->router, part, T, H, E, router_kchunk<CR>(c));
      const float* rbias = c.has_router_bias ? w->router_bias : nullptr;
      if (fused) {  // the chunks' sum, the routing and the group statistics in one launch
        int* gh = (int*)(ws + W.ghist);
        float* gp = (float*)(ws + W.gpart);
        const float tau = c.router_temperature;
        const int nt = c.norm_topk_prob;
        auto go = [&](auto epl) {
          constexpr int EPL = decltype(epl)::value;
          hipLaunchKernelGGL((k_reduce_route<EPL>), dim3(route_groups(T)), dim3(1024), 0, s, part,
                             ns, T, E, k, tau, nt, rbias, st.logits, st.probs, st.lse, st.idx,
                             st.w, gh, gp);
        };
        if (E <= 64) go(std::integral_constant<int, 1>());
        else if (E <= 128) go(std::integral_constant<int, 2>());
        else go(std::integral_constant<int, 4>());
      } else {
        const int64_t TE = (int64_t)T * E;
        hipLaunchKernelGGL(k_router_reduce, dim3(ceil_div(TE, 256)), dim3(256), 0, s, part, ns,
                           TE, E, rbias, st.logits);
      }
    } else {
      using CRN = typename Tilings<D>::RouterNarrow;
      const float* rbias = c.has_router_bias ? w->router_bias : nullptr;
      const int grid = ceil_div(T, CR::BM) * ceil_div(E, CR::BN);
      if (grid < 256) {  // fewer 128-row tiles than CUs
        hipLaunchKernelGGL((k_router_logits<D, CRN>), dim3(ceil_div(T, CRN::BM) * ceil_div(E, CRN::BN)),
                           dim3(CRN::THREADS), 0, s, x, (const D*)w->router, rbias, st.logits, T, H, E);
      } else {
        hipLaunchKernelGGL((k_router_logits<D, CR>), dim3(grid), dim3(CR::THREADS), 0, s, x,
                           (const D*)w->router, rbias, st.logits, T, H, E);
      }
    }
    LAUNCH_CHECK();
  }
  // the fused router's dispatch stops after k_scan; the routed forward's
  // first launch (k_scatter_groups) writes perm and inv_perm
  const bool defer = fused;
  moe_status r = run_routing<D>(p, s, T64, rb, ws, LR, W, &p_join, fused);
  if (r != MOE_OK) return r;
  {
    // beside the dispatch when P is summed on the side stream (the kernel
    // then counts the experts itself), else after the dispatch on s
    const bool side = p_join.armed;
    const hipStream_t ls = side ? p_join.side : s;
    StageTimer tm(p, ls, MOE_STAGE_LOSSES);
    hipLaunchKernelGGL(k_losses, dim3(1), dim3(256), 0, ls, st.P, side ? nullptr : st.counts,
                       st.idx, st.lse, T, E, k, c.aux_switch_coef, c.aux_sqprob_coef, aux, z);
    LAUNCH_CHECK();
  }
  if ((r = routed_fwd<D>(p, s, T, x, st, true, defer ? (const int*)(ws + W.gbase) : nullptr)) !=
      MOE_OK)
    return r;
  HIP_TRY(shared_join.join());
  {
    StageTimer tm(p, s, MOE_STAGE_COMBINE_FWD);
    const int nsl = ceil_div(H / (16 / (int)sizeof(D)), kCombineSlice);
    // the tiled down projection writes Y token-major; the small-token kernel
    // in expert order
    const bool skinny = std::is_same<D, bf16_t>::value && T <= kSkinnyMaxTokens;
    hipLaunchKernelGGL(k_combine_fwd<D>, dim3(ceil_div((int64_t)T * nsl, 4)), dim3(256), 0, s,
                       st.Y, skinny ? st.inv : nullptr,
                       st.w, sY, c.shared_expert_scale, T, k, H, resid, out);
    LAUNCH_CHECK();
  }
  HIP_TRY(p_join.join());  // P and the losses
  return MOE_OK;
}

template <int EPL, typename D>
void launch_router_bwd(hipStream_t s, int grid, const float* probs, const float* lse,
                       const int* idx, const float* w, const float* dw, const float* P,
                       const int* counts, const float* d_aux, const float* d_z, int T, int E,
                       int Epad, int k, const moe_config& c, float* dl, D* dlt) {
  hipLaunchKernelGGL((k_router_bwd<D, EPL>), dim3(grid), dim3(256), 0, s, probs, lse, idx, w, dw,
                     P, counts, d_aux, d_z, T, E, Epad, k, c.router_temperature,
                     c.norm_topk_prob, c.aux_switch_coef, c.aux_sqprob_coef, dl, dlt);
}

template <typename D>
moe_status backward_impl(moe_plan* p, hipStream_t s, int64_t T64, const D* dout,
                         const float* d_aux, const float* d_z, const D* x, const moe_weights* w,
                         const char* saved, char* ws, D* dx, const moe_grads* g,
                         uint8_t* has_grad) {
  using CR = typename Tilings<D>::Router;
  using CB = typename Tilings<D>::Big;
  using CS = WgradTiling<D, 1>;  // grouped weight gradients: single, pair
  using CW = WgradTiling<D, 2>;
  const moe_config& c = p->cfg;
  const int T = (int)T64, H = c.hidden, E = c.num_experts, k = c.experts_per_tok,
            I = c.intermediate, S = c.shared_intermediate;
  const int Epad = round8(E);
  const int64_t TK = T64 * k;
  const WsLayout W = p->ws_layout(T64);
  // With recompute_activations `saved` holds the routing state only: the
  // expert activations are rebuilt in the workspace by the forward's own
  // launches (same kernels, same inputs, so the same bits) before use.
  const bool recompute = c.recompute_activations != 0;
  const SavedLayout LR = p->kept_layout(T64);
  const SavedLayout LA = recompute ? p->saved_layout(T64, moe_plan::Keep::All) : LR;
  char* rb = const_cast<char*>(saved);
  char* ab = recompute ? ws + W.recomp : rb;
  const State<D> st(rb, LR, ab, LA);
  const int* counts = st.counts;
  const int* offsets = st.offsets;
  const int* inv = st.inv;
  const int* idx = st.idx;
  const float* topw = st.w;
  const float* probs = st.probs;
  const float* lse = st.lse;
  const float* P = st.P;
  const D* G = st.G;
  const D* U = st.U;
  const D* A = st.A;
  float* dw = (float*)(ws + W.dw);
  D* dY = (D*)(ws + W.dY);
  D* dG = (D*)(ws + W.dG);
  D* dU = (D*)(ws + W.dU);
  D* dXp = (D*)(ws + W.dXp);
  float* dl = (float*)(ws + W.dlogits);
  D* dlt = (D*)(ws + W.dlogits_t);
  const D* const* tg = (const D* const*)p->d_tab;
  const D* const* tu = (const D* const*)(p->d_tab + E);
  const D* const* td = (const D* const*)(p->d_tab + 2 * E);
  D* const* tdg = (D* const*)(p->d_tab + 3 * E);
  D* const* tdu = (D* const*)(p->d_tab + 4 * E);
  D* const* tdd = (D* const*)(p->d_tab + 5 * E);
  const KGroups kg{offsets, E, 0, 1, 0, TK >= 512 * (int64_t)E ? 1 : 0, nullptr};
  float* partial = (float*)(ws + W.splitk_router);
  // Shared expert backward first, on the plan's second stream: it needs only
  // d_out, x and its own saved activations.  Its input gradient comes first
  // (dx waits for that alone, event sdx), then its weight gradients, which
  // like the routed ones on the third stream are joined only at the end.
  D* dxs = nullptr;
  bool wait_sdx = false;
  SideJoin shared_join, wgrad_join;
  if (S > 0) {
    const hipStream_t ss = p->shared_stream(s);
    HIP_TRY(shared_join.fork(s, ss, p->fork, p->join));
    if (recompute) {
      StageTimer tm(p, ss, MOE_STAGE_RECOMPUTE);
      shared_fwd<D>(p, ss, T, x, w, st.sG, st.sU, st.sA, nullptr);
      LAUNCH_CHECK();
    }
    StageTimer tm(p, ss, MOE_STAGE_SHARED_BWD);
    float* partial_sh = (float*)(ws + W.splitk_shared);
    const D* sG = st.sG;
    const D* sU = st.sU;
    const D* sA = st.sA;
    D* sdG = (D*)(ws + W.sdG);
    D* sdU = (D*)(ws + W.sdU);
    dxs = (D*)(ws + W.dxs);
    const float sc = c.shared_expert_scale;
    const RowGroups dense{nullptr, nullptr, nullptr, nullptr, 1, T, 0, 0};
    with_dense_tiling<D, CB>(T, S, [&](auto c, int grid) {
      using C = decltype(c);
      hipLaunchKernelGGL((k_down_dgrad<D, false, C>), dim3(grid), dim3(C::THREADS), 0, ss, dout,
                         dense, nullptr, (const D*)w->shared_down, H, S, sc, sG, sU, sdG, sdU,
                         nullptr, 0, 1, nullptr);
    });
    with_dense_tiling<D, CB>(T, H, [&](auto c, int grid) {
      using C = decltype(c);
      hipLaunchKernelGGL((k_gateup_dgrad<D, false, C>), dim3(grid), dim3(C::THREADS), 0, ss, sdG,
                         sdU, dense, nullptr, (const D*)w->shared_gate, nullptr,
                         (const D*)w->shared_up, S, H, dxs, nullptr);
    });
    if (ss != s) {
      HIP_TRY(hipEventRecord(p->sdx, ss));
      wait_sdx = true;
    }
    const size_t cap_sh = splitk_bytes<D>(c, T, true);
    moe_status rs = launch_dense_wgrad<D, 1>(ss, dout, nullptr, H, sA, S, T, H, S, sc,
                                             (D*)g->shared_down, nullptr, partial_sh, cap_sh);
    if (rs != MOE_OK) return rs;
    rs = launch_dense_wgrad<D, 2>(ss, sdG, sdU, S, x, H, T, S, H, 1.0f, (D*)g->shared_gate,
                                  (D*)g->shared_up, partial_sh, cap_sh);
    if (rs != MOE_OK) return rs;
  }
  if (recompute) {
    moe_status r = routed_fwd<D>(p, s, T, x, st, false);
    if (r != MOE_OK) return r;
  }
  float* dwp = (float*)(ws + W.dwp);
  // From here the routed weight gradients run on the weight-gradient stream
  // ws2 (they read dY, A, the weighted token rows and, after the down projection's input
  // gradient, dG / dU); the input gradients and the router backward on s.
  const hipStream_t ws2 = p->wgrad_stream(s);
  HIP_TRY(wgrad_join.fork(s, ws2, p->wfork, p->wjoin));
  {
    // the weighted copies of d_out only the down projection's weight
    // gradient reads: beside the input gradient on s
    StageTimer tm(p, ws2, MOE_STAGE_COMBINE_BWD);
    hipLaunchKernelGGL(k_combine_bwd<D>, dim3(ceil_div(T, 4)), dim3(256), 0, ws2, dout, inv,
                       topw, T, k, H, dY);
    LAUNCH_CHECK();
  }
  // whole experts per XCD for the gate/up weight gradient when the experts
  // split evenly over the XCDs (k_xcd_order decides on the device)
  int* xorder = E % 8 == 0 ? (int*)(ws + W.xorder) : nullptr;
  if (p->xflag_pending && hipEventQuery(p->xflag_ev) == hipSuccess) {
    p->xflag = *p->h_xflag;
    p->xflag_pending = false;
  }
  const bool expect_whole = xorder && p->xflag == 1;
  if (xorder) {
    hipLaunchKernelGGL(k_xcd_order, dim3(1), dim3(1024), 0, ws2, counts, E, xorder);
    LAUNCH_CHECK();
    if (!p->xflag_pending && p->h_xflag) {
      HIP_TRY(hipMemcpyAsync(p->h_xflag, xorder + E, sizeof(int), hipMemcpyDeviceToHost, ws2));
      HIP_TRY(hipEventRecord(p->xflag_ev, ws2));
      p->xflag_pending = true;
    }
  }
  {
    StageTimer tm(p, ws2, MOE_STAGE_DOWN_WGRAD);
    const int grid = kgrouped_grid(E, H, I, CS::BM, CS::BN);
    // the down projection's weight gradient walks its tiles down columns for
    // every group size (config 5's ~256-row groups: 3.52 -> 3.42 ms in a
    // probe; the gate/up pair keeps the size rule of kg)
    KGroups kgd = kg;
    kgd.col_walk = 1;
    hipLaunchKernelGGL((k_wgrad<D, 1, true>), dim3(grid), dim3(CS::THREADS), 0, ws2, dY, nullptr, (int64_t)H, A,
                       (int64_t)I, kgd, H, I, 1.0f, tdd, nullptr, nullptr, nullptr, nullptr, grid, 0);
    LAUNCH_CHECK();
  }
  {
    StageTimer tm(p, s, MOE_STAGE_DOWN_DGRAD);
    with_row_tiling<D, CB, false>(offsets, st.tprefix, E, TK, [&](auto c, const RowGroups& r, auto grid) {
      using C = decltype(c);
      hipLaunchKernelGGL((k_down_dgrad<D, true, C>), dim3(grid(I)), dim3(C::THREADS), 0, s,
                         dout, r, td, nullptr, H, I, 1.0f, G, U, dG, dU, st.perm, T, k, dwp);
    });
    LAUNCH_CHECK();
    hipLaunchKernelGGL(k_dw_sum, dim3(ceil_div(TK, (int64_t)256)), dim3(256), 0, s, dwp,
                       ceil_div(I, 32), (int)TK, st.perm, dw);
    LAUNCH_CHECK();
  }
  // the gate/up weight gradient's token rows, weighted (its dG_u, dU_u leave
  // the routing weight out), in dY's region once the down projection's
  // weight gradient has read it (same stream).  Launched after the input
  // gradient on s, so a serial run (one stream) keeps the order of the
  // overlapped one for the caches: d_out rows, G and U are read first.
  D* xw = dY;
  {
    StageTimer tm(p, ws2, MOE_STAGE_GATHER);
    hipLaunchKernelGGL(k_gather<D>, dim3(ceil_div(T, 4)), dim3(256), 0, ws2, x, inv, T, k, H, xw,
                       topw);
    LAUNCH_CHECK();
  }
  if (ws2 != s) {
    HIP_TRY(hipEventRecord(p->wmid, s));
    HIP_TRY(hipStreamWaitEvent(ws2, p->wmid, 0));
  }
  {
    StageTimer tm(p, ws2, MOE_STAGE_GATEUP_WGRAD);
    const int grid = kgrouped_grid(E, I, H, CW::BM, CW::BN);
    KGroups kgp = kg;
    kgp.xcd_order = xorder;
    const int slots = std::min(grid, p->wgrad_slots);
    hipLaunchKernelGGL((k_wgrad<D, 2, true>), dim3(expect_whole ? slots : grid), dim3(CW::THREADS), 0, ws2, dG, dU, (int64_t)I, xw,
                       (int64_t)H, kgp, I, H, 1.0f, tdg, nullptr, tdu, nullptr, nullptr, grid,
                       slots);
    LAUNCH_CHECK();
  }
  {
    StageTimer tm(p, s, MOE_STAGE_GATEUP_DGRAD);
    with_row_tiling<D, CB>(offsets, st.tprefix, E, TK, [&](auto c, const RowGroups& r, auto grid) {
      using C = decltype(c);
      hipLaunchKernelGGL((k_gateup_dgrad<D, true, C>), dim3(grid(H)), dim3(C::THREADS), 0,
                         s, dG, dU, r, tg, nullptr, tu, nullptr, I, H, dXp, st.perm);
    });
    LAUNCH_CHECK();
  }
  {
    StageTimer tm(p, s, MOE_STAGE_ROUTER_BWD);
    const int grid = ceil_div(T, 4);
    switch (route_epl(E)) {
      case 1: launch_router_bwd<1, D>(s, grid, probs, lse, idx, topw, dw, P, counts, d_aux, d_z, T, E, Epad, k, c, dl, dlt); break;
      case 2: launch_router_bwd<2, D>(s, grid, probs, lse, idx, topw, dw, P, counts, d_aux, d_z, T, E, Epad, k, c, dl, dlt); break;
      case 4: launch_router_bwd<4, D>(s, grid, probs, lse, idx, topw, dw, P, counts, d_aux, d_z, T, E, Epad, k, c, dl, dlt); break;
      case 8: launch_router_bwd<8, D>(s, grid, probs, lse, idx, topw, dw, P, counts, d_aux, d_z, T, E, Epad, k, c, dl, dlt); break;
      default: launch_router_bwd<16, D>(s, grid, probs, lse, idx, topw, dw, P, counts, d_aux, d_z, T, E, Epad, k, c, dl, dlt); break;
    }
    LAUNCH_CHECK();
    const moe_status rr = launch_dense_wgrad<D, 1>(s, dlt, nullptr, Epad, x, H, T, E, H, 1.0f,
                                                   (D*)g->router, nullptr, partial,
                                                   splitk_bytes<D>(c, T, false));
    if (rr != MOE_OK) return rr;
    if (c.has_router_bias && g->router_bias) {
      const int nrb = colsum_rows(T, false);
      float* part = (float*)(ws);  // column partials at workspace offset 0
      hipLaunchKernelGGL(k_colsum_partial, dim3(ceil_div(E, 64), nrb), dim3(256), 0, s, dl, T, E,
                         part);
      hipLaunchKernelGGL(k_colsum_final, dim3(ceil_div(E, 256)), dim3(256), 0, s, part, nrb, E,
                         1.0f, g->router_bias);
    }
    LAUNCH_CHECK();
  }
  // dx reads dXp and the router gradient (this stream) and the shared dx: the
  // weight-gradient kernels still running on the side streams are joined after it
  if (wait_sdx) HIP_TRY(hipStreamWaitEvent(s, p->sdx, 0));
  {
    StageTimer tm(p, s, MOE_STAGE_DX);
    using CX = typename Tilings<D>::RouterDx;
    const dim3 grid(ceil_div(T, CX::BM) * ceil_div(H, CX::BN));
    const D* wr = (const D*)w->router;
    if (k <= 2)
      hipLaunchKernelGGL((k_router_dgrad<D, 2>), grid, dim3(256), 0, s, dlt, Epad, E, wr, T, H, dXp, nullptr, k, topw, dxs, dx);
    else if (k <= 4)
      hipLaunchKernelGGL((k_router_dgrad<D, 4>), grid, dim3(256), 0, s, dlt, Epad, E, wr, T, H, dXp, nullptr, k, topw, dxs, dx);
    else if (k <= 8)
      hipLaunchKernelGGL((k_router_dgrad<D, 8>), grid, dim3(256), 0, s, dlt, Epad, E, wr, T, H, dXp, nullptr, k, topw, dxs, dx);
    else
      hipLaunchKernelGGL((k_router_dgrad<D, 16>), grid, dim3(256), 0, s, dlt, Epad, E, wr, T, H, dXp, nullptr, k, topw, dxs, dx);
    if (has_grad) hipLaunchKernelGGL(k_has_grad, dim3(ceil_div(E, 256)), dim3(256), 0, s, counts, E, has_grad);
    LAUNCH_CHECK();
  }
  HIP_TRY(wgrad_join.join());
  HIP_TRY(shared_join.join());
  return MOE_OK;
}

// Device addresses of `scratch`, one per device, resolved once per device
// (with that device current) and kept for the life of the process.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

moe_status resolve_scratch(int device, void** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device < 0 || device >= kMaxScratchDevices)
    return fail(MOE_ERR_UNSUPPORTED, "device %d: no static scratch slot", device);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(MOE_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                  hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return MOE_OK;
}

moe_status check_plan(const moe_plan* p) {
  if (!p) return fail(MOE_ERR_INVALID, "plan is NULL");
  return MOE_OK;
}

moe_status validate_config(const moe_config* c) {
  if (!c) return fail(MOE_ERR_INVALID, "config is NULL");
  if (c->dtype != MOE_DTYPE_F32 && c->dtype != MOE_DTYPE_BF16)
    return fail(MOE_ERR_INVALID, "dtype %d is not MOE_DTYPE_F32 or MOE_DTYPE_BF16", c->dtype);
  if (c->hidden <= 0 || c->hidden % 8)
    return fail(MOE_ERR_INVALID, "hidden (%d) must be a positive multiple of 8", c->hidden);
  if (c->intermediate <= 0)
    return fail(MOE_ERR_INVALID, "MoE cfg.moe.intermediate_size must be non-zero");
  if (c->intermediate % 8)
    return fail(MOE_ERR_INVALID, "intermediate_size (%d) must be a multiple of 8", c->intermediate);
  if (c->shared_intermediate < 0 || c->shared_intermediate % 8)
    return fail(MOE_ERR_INVALID, "shared_intermediate (%d) must be 0 or a multiple of 8",
                c->shared_intermediate);
  if (c->num_experts < 1 || c->num_experts > 1024)
    return fail(MOE_ERR_INVALID, "num_experts (%d) must be in 1..1024", c->num_experts);
  if (c->experts_per_tok < 1)
    return fail(MOE_ERR_INVALID, "experts_per_tok (%d) must be at least 1", c->experts_per_tok);
  if (c->experts_per_tok > c->num_experts)
    return fail(MOE_ERR_INVALID, "MoE experts_per_tok (%d) must not exceed num_experts (%d)",
                c->experts_per_tok, c->num_experts);
  if (c->experts_per_tok > 16)
    return fail(MOE_ERR_UNSUPPORTED, "experts_per_tok (%d) above 16 is not supported",
                c->experts_per_tok);
  if (!(c->router_temperature > 0.0f))
    return fail(MOE_ERR_INVALID, "router_temperature must be positive");
  if (c->recompute_activations != 0 && c->recompute_activations != 1)
    return fail(MOE_ERR_INVALID, "recompute_activations (%d) must be 0 or 1",
                c->recompute_activations);
  if (c->fused_block != 0 && c->fused_block != 1)
    return fail(MOE_ERR_INVALID, "fused_block (%d) must be 0 or 1", c->fused_block);
  if (c->fused_block && !(c->rms_norm_eps >= 0.0f))
    return fail(MOE_ERR_INVALID, "rms_norm_eps must be non-negative");
  if (c->fused_block && c->hidden > 8192)
    return fail(MOE_ERR_UNSUPPORTED, "fused_block supports hidden <= 8192 (got %d)", c->hidden);
  // every weight matrix is read through one buffer resource (32-bit offsets)
  const int64_t wide = std::max<int64_t>({c->intermediate, c->shared_intermediate,
                                          round8(c->num_experts)});
  if (wide * c->hidden * elt_size(c->dtype) >= kMaxExtentBytes)
    return fail(MOE_ERR_UNSUPPORTED,
                "a weight matrix of %lld x %d elements reaches 2^31 bytes (32-bit buffer offsets)",
                (long long)wide, c->hidden);
  return MOE_OK;
}

// Largest buffer-resource extent of a call over T tokens, in bytes.  Operand
// tiles start at their own rows, so an extent spans the rows (or, for a weight
// gradient, the reduction rows) of one group: an expert holds at most T rows,
// since a token picks k distinct experts.  The widest row is H, I, S or the
// padded expert count of the router's logit gradient.
int64_t max_token_extent(const moe_config& c, int64_t T) {
  const int64_t wide = std::max<int64_t>({c.hidden, c.intermediate, c.shared_intermediate,
                                          round8(c.num_experts)});
  return T * wide * elt_size(c.dtype);
}

moe_status check_tokens_cfg(const moe_config& c, int64_t T) {
  if (T < 0) return fail(MOE_ERR_INVALID, "num_tokens (%lld) is negative", (long long)T);
  if (T > (1 << 24)) return fail(MOE_ERR_UNSUPPORTED, "num_tokens (%lld) above 2^24", (long long)T);
  if (max_token_extent(c, T) >= kMaxExtentBytes)
    return fail(MOE_ERR_UNSUPPORTED,
                "num_tokens (%lld): a %lld-byte operand reaches 2^31 bytes (32-bit buffer "
                "offsets); split the batch",
                (long long)T, (long long)max_token_extent(c, T));
  return MOE_OK;
}

moe_status check_tokens(const moe_plan* p, int64_t T) { return check_tokens_cfg(p->cfg, T); }

// The workspace plan of a call over T tokens against what its launches need,
// without a device: every region a launch writes or reads (sized from the
// same helpers the launches take their grids and splits from: hist_blocks,
// route_groups, colsum_rows, router_path, dense_wgrad_partial_bytes,
// norm_tree, the saved layouts) must fit the region ws_layout gives it, the
// regions of one phase must not overlap, and every region must lie inside the
// workspace (the forward's inside its forward part, which bounds the static
// scratch of moe_forward_noalloc).
template <typename D>
moe_status check_workspace_plan(const moe_plan& p, int64_t T) {
  const moe_config& c = p.cfg;
  const int E = c.num_experts, k = c.experts_per_tok, H = c.hidden, I = c.intermediate,
            S = c.shared_intermediate;
  const int64_t TK = T * k;
  const size_t b = sizeof(D);
  const WsLayout W = p.ws_layout(T);
  struct Need { const char* name; size_t bytes; };
  Need need[kMaxWsSpans];
  int n = 0;
  auto add = [&](const char* name, size_t bytes) {
    if (n < kMaxWsSpans) need[n++] = {name, bytes};
  };
  if (T > 0) {
    const RouterPath rp = router_path(c, T);
    const bool fused = group_routing(c, T);
    if (T > kRouteSmallTokens) {
      if (!fused) {
        add("block_hist", 4 * (size_t)hist_blocks(T) * E);
        add("block_base", 4 * (size_t)hist_blocks(T) * E);
      } else {
        add("ghist", 4 * (size_t)route_groups(T) * E);
        add("gbase", 4 * (size_t)route_groups(T) * E);
        add("gpart", 4 * (size_t)route_groups(T) * E);
      }
      add("colpart", 4 * (size_t)colsum_rows(T, fused) * E);
    }
    if (rp == RouterPath::Split) add("rpart", 4 * (size_t)router_splits(c) * T * E);
    if (S > 0) add("sY", b * T * H);
    add("infer", p.saved_layout(T, moe_plan::Keep::Transient).total);
    if (c.has_router_bias) add("bias_colpart", 4 * (size_t)colsum_rows(T, false) * E);
    add("dw", 4 * TK);
    add("dwp", 4 * (size_t)ceil_div(I, 32) * TK);
    add("dY", b * TK * H);
    add("dG", b * TK * I);
    add("dU", b * TK * I);
    add("dXp", b * TK * H);
    add("dlogits", 4 * T * E);
    add("dlogits_t", b * T * round8(E));
    add("splitk_router", dense_wgrad_partial_bytes<D, 1>(E, H, (int)T));
    if (S > 0) {
      add("sdG", b * T * S);
      add("sdU", b * T * S);
      add("dxs", b * T * H);
      add("splitk_shared", std::max(dense_wgrad_partial_bytes<D, 1>(H, S, (int)T),
                                    dense_wgrad_partial_bytes<D, 2>(S, H, (int)T)));
    }
    if (c.recompute_activations) add("recomp", p.saved_layout(T, moe_plan::Keep::All).total);
    if (c.fused_block) {
      const int nrow = ceil_div(T, kRmsRows);
      size_t rows[2] = {0, 0};
      norm_tree(nrow, [&](int, int G, int which) {
        rows[which] = std::max(rows[which], (size_t)G);
      });
      add("dxm", b * T * H);
      add("dwn", 4 * (size_t)nrow * H);
      add("dwn_a", 4 * rows[0] * H);
      add("dwn_b", 4 * rows[1] * H);
    }
    if (E % 8 == 0) add("xorder", 4 * (size_t)(E + 1));
  }
  if (n >= kMaxWsSpans || W.nspan >= kMaxWsSpans)
    return fail(MOE_ERR_INVALID, "workspace check: more regions than it records");
  for (int i = 0; i < n; ++i) {
    const WsSpan* sp = nullptr;
    for (int j = 0; j < W.nspan; ++j)
      if (strcmp(W.span[j].name, need[i].name) == 0) sp = &W.span[j];
    if (!sp) return fail(MOE_ERR_INVALID, "workspace check: no region %s", need[i].name);
    if (need[i].bytes > sp->bytes)
      return fail(MOE_ERR_INVALID,
                  "workspace check: T = %lld needs %zu bytes in region %s, which holds %zu",
                  (long long)T, need[i].bytes, need[i].name, sp->bytes);
  }
  for (int i = 0; i < W.nspan; ++i) {
    const WsSpan& a = W.span[i];
    const size_t end = a.off + a.bytes;
    if (end > W.total || (a.phase == 0 && end > W.fwd_total))
      return fail(MOE_ERR_INVALID, "workspace check: region %s [%zu, %zu) outside the workspace",
                  a.name, a.off, end);
    for (int j = 0; j < W.nspan; ++j) {
      const WsSpan& o = W.span[j];
      if (j == i || o.phase != a.phase || a.bytes == 0 || o.bytes == 0) continue;
      if (a.off < o.off + o.bytes && o.off < end)
        return fail(MOE_ERR_INVALID, "workspace check: regions %s and %s overlap", a.name, o.name);
    }
  }
  return MOE_OK;
}

}  // namespace

extern "C" {

void moe_config_default(moe_config* cfg, int32_t hidden, int32_t num_experts,
                        int32_t experts_per_tok, int32_t intermediate,
                        int32_t shared_intermediate) {
  if (!cfg) return;
  memset(cfg, 0, sizeof(*cfg));
  cfg->hidden = hidden;
  cfg->num_experts = num_experts;
  cfg->experts_per_tok = experts_per_tok;
  cfg->intermediate = intermediate;
  cfg->shared_intermediate = shared_intermediate;
  cfg->dtype = MOE_DTYPE_BF16;
  cfg->router_temperature = 1.0f;
  cfg->shared_expert_scale = 1.0f;
  cfg->aux_switch_coef = 1.0f;
  cfg->aux_sqprob_coef = 1.0f;
}

moe_status moe_plan_create(const moe_config* cfg, int device, moe_plan** out) {
  if (!out) return fail(MOE_ERR_INVALID, "plan output pointer is NULL");
  *out = nullptr;
  moe_status st = validate_config(cfg);
  if (st != MOE_OK) return st;
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(MOE_ERR_INVALID, "device %d out of range (%d)", device, n);
  HIP_TRY(hipSetDevice(device));
  moe_plan* p = new (std::nothrow) moe_plan();
  if (!p) return fail(MOE_ERR_OOM, "host allocation of the plan failed");
  p->cfg = *cfg;
  p->device = device;
  {
    int ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
        ncu >= 8)
      p->wgrad_slots = ncu / 8 * 8;
  }
  // the static scratch of moe_forward_noalloc on this device (device current)
  if (resolve_scratch(device, &p->scratch_ptr) != MOE_OK) {
    delete p;
    return MOE_ERR_HIP;
  }
  const size_t tab_bytes = sizeof(void*) * 6 * (size_t)cfg->num_experts;
  hipError_t e = hipMalloc((void**)&p->d_tab, tab_bytes);
  if (e == hipSuccess)
    e = hipHostMalloc((void**)&p->h_tab, tab_bytes * moe_plan::kTabSlots, hipHostMallocDefault);
  if (e == hipSuccess) e = hipMemset(p->d_tab, 0, tab_bytes);
  for (int i = 0; i < moe_plan::kTabSlots && e == hipSuccess; ++i)
    e = hipEventCreateWithFlags(&p->tab_ev[i], hipEventDisableTiming);
  if (e == hipSuccess && cfg->shared_intermediate > 0) {
    e = hipStreamCreateWithFlags(&p->aux, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->join, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->sdx, hipEventDisableTiming);
  }
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->wgs, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->wfork, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->wmid, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->wjoin, hipEventDisableTiming);
  if (e == hipSuccess) e = hipHostMalloc((void**)&p->h_xflag, sizeof(int), hipHostMallocDefault);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->xflag_ev, hipEventDisableTiming);
  if (e != hipSuccess) {
    moe_plan_destroy(p);
    return fail(e == hipErrorOutOfMemory ? MOE_ERR_OOM : MOE_ERR_HIP, "plan set-up: %s",
                hipGetErrorString(e));
  }
  *out = p;
  return MOE_OK;
}

moe_status moe_plan_destroy(moe_plan* p) {
  if (!p) return MOE_OK;
  // teardown: nothing to report if a release fails
  for (auto& q : p->pending) {
    (void)hipEventSynchronize(q.b);
    (void)hipEventDestroy(q.a);
    (void)hipEventDestroy(q.b);
  }
  for (auto e : p->free_events) (void)hipEventDestroy(e);
  if (p->aux) (void)hipStreamSynchronize(p->aux);
  if (p->fork) (void)hipEventDestroy(p->fork);
  if (p->join) (void)hipEventDestroy(p->join);
  if (p->sdx) (void)hipEventDestroy(p->sdx);
  if (p->aux) (void)hipStreamDestroy(p->aux);
  if (p->wgs) (void)hipStreamSynchronize(p->wgs);
  for (hipEvent_t ev : {p->wfork, p->wmid, p->wjoin})
    if (ev) (void)hipEventDestroy(ev);
  if (p->wgs) (void)hipStreamDestroy(p->wgs);
  for (int i = 0; i < moe_plan::kTabSlots; ++i) {
    if (!p->tab_ev[i]) continue;
    if (p->tab_ev_pending[i]) (void)hipEventSynchronize(p->tab_ev[i]);
    (void)hipEventDestroy(p->tab_ev[i]);
  }
  if (p->d_tab) (void)hipFree(p->d_tab);
  if (p->h_tab) (void)hipHostFree(p->h_tab);
  if (p->xflag_ev) {
    if (p->xflag_pending) (void)hipEventSynchronize(p->xflag_ev);
    (void)hipEventDestroy(p->xflag_ev);
  }
  if (p->h_xflag) (void)hipHostFree(p->h_xflag);
  delete p;
  return MOE_OK;
}

moe_status moe_check_tokens(const moe_config* cfg, int64_t T) {
  moe_status st = validate_config(cfg);
  if (st != MOE_OK) return st;
  return check_tokens_cfg(*cfg, T);
}

moe_status moe_workspace_check(const moe_config* cfg, int64_t T) {
  moe_status st = validate_config(cfg);
  if (st != MOE_OK) return st;
  if ((st = check_tokens_cfg(*cfg, T)) != MOE_OK) return st;
  moe_plan plan;  // layout arithmetic only: no device resources
  plan.cfg = *cfg;
  return cfg->dtype == MOE_DTYPE_BF16 ? check_workspace_plan<bf16_t>(plan, T)
                                      : check_workspace_plan<float>(plan, T);
}

size_t moe_saved_bytes(const moe_plan* p, int64_t T) {
  if (!p || T < 0) return 0;
  return p->kept_layout(T).total;
}

size_t moe_workspace_bytes(const moe_plan* p, int64_t T) {
  if (!p || T < 0) return 0;
  return p->ws_layout(T).total;
}

moe_status moe_saved_field_range(const moe_plan* p, int64_t T, int32_t field, size_t* offset,
                                 size_t* bytes) {
  if (!p) return fail(MOE_ERR_INVALID, "plan is NULL");
  if (field < 0 || field >= MOE_SAVED_NUM_FIELDS)
    return fail(MOE_ERR_INVALID, "unknown saved field %d", field);
  const SavedLayout L = p->kept_layout(T);
  if (offset) *offset = L.f[field];
  if (bytes) *bytes = L.fbytes[field];
  return MOE_OK;
}

}  // extern "C"

namespace {

// RMSNorm forward of the block path into (xn, rstd).
template <typename D>
void launch_norm_fwd(moe_plan* p, hipStream_t s, int T, const void* h, const void* nw, char* xn,
                     float* rstd) {
  StageTimer tm(p, s, MOE_STAGE_NORM_FWD);
  hipLaunchKernelGGL(k_rmsnorm_fwd<D>, dim3(ceil_div(T, 4)), dim3(256), 0, s, (const D*)h,
                     (const D*)nw, p->cfg.rms_norm_eps, T, p->cfg.hidden, (D*)xn, rstd);
}

// RMSNorm backward of the block path: dh and the weight gradient (partial
// rows per kRmsRows tokens, then a fixed 16-ary reduction tree).
template <typename D>
void launch_norm_bwd(moe_plan* p, hipStream_t s, int T, const D* dxm, const void* h,
                     const void* nw, const float* rstd, const void* dout, void* dh, void* dnw,
                     char* ws, const WsLayout& W) {
  StageTimer tm(p, s, MOE_STAGE_NORM_BWD);
  const int H = p->cfg.hidden;
  const int nrow = ceil_div(T, kRmsRows);
  float* part = (float*)(ws + W.dwn);
  auto bwd = [&](auto nch) {
    constexpr int NCH = decltype(nch)::value;
    hipLaunchKernelGGL((k_rmsnorm_bwd<D, NCH>), dim3(nrow), dim3(256), 0, s, dxm, (const D*)h,
                       (const D*)nw, rstd, (const D*)dout, T, H, (D*)dh, part);
  };
  if (H <= 2048) bwd(std::integral_constant<int, 1>());
  else if (H <= 4096) bwd(std::integral_constant<int, 2>());
  else bwd(std::integral_constant<int, 4>());
  const float* in = part;
  float* bufs[2] = {(float*)(ws + W.dwn_a), (float*)(ws + W.dwn_b)};
  int R = nrow;
  norm_tree(nrow, [&](int r, int G, int which) {
    hipLaunchKernelGGL(k_rowsum<float>, dim3(ceil_div(H, 2048), G), dim3(256), 0, s, in, r, H,
                       16, bufs[which]);
    in = bufs[which];
    R = G;
  });
  hipLaunchKernelGGL(k_rowsum<D>, dim3(ceil_div(H, 2048), 1), dim3(256), 0, s, in, R, H, R,
                     (D*)dnw);
}

// Shared argument checks and table upload of the forward entry points.
// block: moe_block_forward (x is h, nw the RMSNorm weight).
moe_status forward_entry(moe_plan* p, void* stream, int64_t T, const void* x, const void* nw,
                         const moe_weights* w, void* out, float* aux_loss, float* z_loss,
                         void* saved, void* workspace, bool block) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  if ((st = check_tokens(p, T)) != MOE_OK) return st;
  if (!w) return fail(MOE_ERR_INVALID, "weights struct is NULL");
  const moe_config& c = p->cfg;
  if (block && !c.fused_block)
    return fail(MOE_ERR_INVALID, "moe_block_forward needs a plan created with fused_block = 1");
  if (!block && c.fused_block)
    return fail(MOE_ERR_INVALID, "the plan was created with fused_block = 1: call moe_block_forward");
  if (T > 0 && (!x || !out || !workspace || !w->router || !w->gate || !w->up || !w->down ||
                (block && !nw)))
    return fail(MOE_ERR_INVALID, "a required pointer is NULL");
  if (c.has_router_bias && !w->router_bias)
    return fail(MOE_ERR_INVALID, "has_router_bias is set but router_bias is NULL");
  if (c.shared_intermediate > 0 && (!w->shared_gate || !w->shared_up || !w->shared_down))
    return fail(MOE_ERR_INVALID, "shared expert enabled but its weights are NULL");
  const void* ptrs[] = {x, nw, out, saved, workspace, w->router, w->shared_gate, w->shared_up,
                        w->shared_down};
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(MOE_ERR_INVALID, "device pointers must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipSetDevice(p->device));
  if (T == 0) {
    if ((st = zero_async(s, aux_loss, sizeof(float))) != MOE_OK) return st;
    return zero_async(s, z_loss, sizeof(float));
  }
  const void* const* tabs[3] = {w->gate, w->up, w->down};
  if ((st = upload_tables(p, s, 0, tabs)) != MOE_OK) return st;
  const bool bf = c.dtype == MOE_DTYPE_BF16;
  const void* xin = x;
  const void* resid = nullptr;
  if (block) {
    // x = RMSNorm(h): kept in `saved`, or transient in the workspace
    const bool keep_act = saved && !c.recompute_activations;
    const WsLayout W = p->ws_layout(T);
    const SavedLayout LA =
        keep_act ? p->kept_layout(T) : p->saved_layout(T, moe_plan::Keep::Transient);
    char* ab = keep_act ? (char*)saved : (char*)workspace + W.infer;
    char* xn = ab + LA.f[MOE_SAVED_NORM_X];
    float* rstd = (float*)(ab + LA.f[MOE_SAVED_RSTD]);
    if (bf) launch_norm_fwd<bf16_t>(p, s, (int)T, x, nw, xn, rstd);
    else launch_norm_fwd<float>(p, s, (int)T, x, nw, xn, rstd);
    LAUNCH_CHECK();
    xin = xn;
    resid = x;
  }
  if (bf)
    return forward_impl<bf16_t>(p, s, T, (const bf16_t*)xin, w, (bf16_t*)out, aux_loss, z_loss,
                                (char*)saved, (char*)workspace, (const bf16_t*)resid);
  return forward_impl<float>(p, s, T, (const float*)xin, w, (float*)out, aux_loss, z_loss,
                             (char*)saved, (char*)workspace, (const float*)resid);
}

moe_status backward_entry(moe_plan* p, void* stream, int64_t T, const void* d_out,
                          const float* d_aux, const float* d_z, const void* x, const void* nw,
                          const moe_weights* w, const void* saved, void* workspace, void* dx,
                          void* dnw, const moe_grads* g, uint8_t* has_grad, bool block) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  if ((st = check_tokens(p, T)) != MOE_OK) return st;
  if (!w || !g) return fail(MOE_ERR_INVALID, "weights or grads struct is NULL");
  const moe_config& c = p->cfg;
  if (block && !c.fused_block)
    return fail(MOE_ERR_INVALID, "moe_block_backward needs a plan created with fused_block = 1");
  if (!block && c.fused_block)
    return fail(MOE_ERR_INVALID, "the plan was created with fused_block = 1: call moe_block_backward");
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipSetDevice(p->device));
  if (T == 0) {
    // No token: no expert has a gradient entry (has_grad all 0, expert
    // buffers untouched), and the dense gradients are sums over no token.
    const size_t b = elt_size(c.dtype), H = c.hidden, E = c.num_experts,
                 S = c.shared_intermediate;
    const std::pair<void*, size_t> clear[] = {
        {has_grad, E}, {g->router, E * H * b}, {g->router_bias, c.has_router_bias ? E * 4 : 0},
        {g->shared_gate, S * H * b}, {g->shared_up, S * H * b}, {g->shared_down, H * S * b},
        {block ? dnw : nullptr, H * b}};
    for (const auto& q : clear)
      if ((st = zero_async(s, q.first, q.second)) != MOE_OK) return st;
    return MOE_OK;
  }
  if (!d_out || !x || !saved || !workspace || !dx || !w->router || !w->gate || !w->up ||
      !w->down || !g->router || !g->gate || !g->up || !g->down || (block && (!nw || !dnw)))
    return fail(MOE_ERR_INVALID, "a required pointer is NULL");
  if (c.shared_intermediate > 0 &&
      (!w->shared_gate || !w->shared_up || !w->shared_down || !g->shared_gate || !g->shared_up ||
       !g->shared_down))
    return fail(MOE_ERR_INVALID, "shared expert enabled but its weights or grads are NULL");
  const void* ptrs[] = {d_out, x, nw, dnw, saved, workspace, dx, w->router, g->router,
                        g->shared_gate, g->shared_up, g->shared_down};
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(MOE_ERR_INVALID, "device pointers must be 16-byte aligned");
  const void* const* tabs[3] = {w->gate, w->up, w->down};
  if ((st = upload_tables(p, s, 0, tabs)) != MOE_OK) return st;
  const void* const* gtabs[3] = {(const void* const*)g->gate, (const void* const*)g->up,
                                 (const void* const*)g->down};
  if ((st = upload_tables(p, s, 3, gtabs)) != MOE_OK) return st;
  const bool bf = c.dtype == MOE_DTYPE_BF16;
  const WsLayout W = p->ws_layout(T);
  const void* xin = x;
  void* dxo = dx;
  const float* rstd = nullptr;
  if (block) {
    // the layer's input x = RMSNorm(h): kept, or rebuilt with the forward's kernel
    const bool recompute = c.recompute_activations != 0;
    const SavedLayout LA =
        recompute ? p->saved_layout(T, moe_plan::Keep::All) : p->kept_layout(T);
    char* ab = recompute ? (char*)workspace + W.recomp : (char*)saved;
    char* xn = ab + LA.f[MOE_SAVED_NORM_X];
    rstd = (const float*)(ab + LA.f[MOE_SAVED_RSTD]);
    if (recompute) {
      if (bf) launch_norm_fwd<bf16_t>(p, s, (int)T, x, nw, xn, (float*)rstd);
      else launch_norm_fwd<float>(p, s, (int)T, x, nw, xn, (float*)rstd);
      LAUNCH_CHECK();
    }
    xin = xn;
    dxo = (char*)workspace + W.dxm;
  }
  if (bf)
    st = backward_impl<bf16_t>(p, s, T, (const bf16_t*)d_out, d_aux, d_z, (const bf16_t*)xin, w,
                               (const char*)saved, (char*)workspace, (bf16_t*)dxo, g, has_grad);
  else
    st = backward_impl<float>(p, s, T, (const float*)d_out, d_aux, d_z, (const float*)xin, w,
                              (const char*)saved, (char*)workspace, (float*)dxo, g, has_grad);
  if (st != MOE_OK || !block) return st;
  if (bf)
    launch_norm_bwd<bf16_t>(p, s, (int)T, (const bf16_t*)dxo, x, nw, rstd, d_out, dx, dnw,
                            (char*)workspace, W);
  else
    launch_norm_bwd<float>(p, s, (int)T, (const float*)dxo, x, nw, rstd, d_out, dx, dnw,
                           (char*)workspace, W);
  LAUNCH_CHECK();
  return MOE_OK;
}

}  // namespace

extern "C" {

moe_status moe_forward(moe_plan* p, void* stream, int64_t T, const void* x, const moe_weights* w,
                       void* out, float* aux_loss, float* z_loss, void* saved, void* workspace) {
  return forward_entry(p, stream, T, x, nullptr, w, out, aux_loss, z_loss, saved, workspace,
                       false);
}

moe_status moe_block_forward(moe_plan* p, void* stream, int64_t T, const void* h,
                             const void* norm_weight, const moe_weights* w, void* out,
                             float* aux_loss, float* z_loss, void* saved, void* workspace) {
  return forward_entry(p, stream, T, h, norm_weight, w, out, aux_loss, z_loss, saved, workspace,
                       true);
}

moe_status moe_backward(moe_plan* p, void* stream, int64_t T, const void* d_out,
                        const float* d_aux, const float* d_z, const void* x,
                        const moe_weights* w, const void* saved, void* workspace, void* dx,
                        const moe_grads* g, uint8_t* has_grad) {
  return backward_entry(p, stream, T, d_out, d_aux, d_z, x, nullptr, w, saved, workspace, dx,
                        nullptr, g, has_grad, false);
}

moe_status moe_block_backward(moe_plan* p, void* stream, int64_t T, const void* d_out,
                              const float* d_aux, const float* d_z, const void* h,
                              const void* norm_weight, const moe_weights* w, const void* saved,
                              void* workspace, void* dh, void* d_norm_weight, const moe_grads* g,
                              uint8_t* has_grad) {
  return backward_entry(p, stream, T, d_out, d_aux, d_z, h, norm_weight, w, saved, workspace,
                        dh, d_norm_weight, g, has_grad, true);
}

moe_status moe_forward_noalloc(moe_plan* p, void* stream, int64_t T, const void* x,
                               const moe_weights* w, void* out, float* aux_loss, float* z_loss) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  if ((st = check_tokens(p, T)) != MOE_OK) return st;
  if (!p->scratch_ptr) return fail(MOE_ERR_HIP, "the plan has no static scratch");
  const size_t need = p->ws_layout(T).fwd_total;
  if (need > kNoAllocScratchBytes)
    return fail(MOE_ERR_UNSUPPORTED,
                "moe_forward_noalloc: %lld tokens need %zu bytes of scratch, above the %zu-byte "
                "static scratch; call moe_forward with a workspace",
                (long long)T, need, kNoAllocScratchBytes);
  // no per-stage events: creating them could allocate
  const uint32_t mask = p->profile_mask;
  p->profile_mask = 0;
  st = forward_entry(p, stream, T, x, nullptr, w, out, aux_loss, z_loss, nullptr, p->scratch_ptr,
                     false);
  p->profile_mask = mask;
  return st;
}

moe_status moe_route_from_logits(moe_plan* p, void* stream, int64_t T, const float* logits,
                                 void* saved, void* workspace) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  if ((st = check_tokens(p, T)) != MOE_OK) return st;
  if (T == 0) return MOE_OK;
  if (!logits || !saved || !workspace) return fail(MOE_ERR_INVALID, "a required pointer is NULL");
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipSetDevice(p->device));
  const SavedLayout L = p->kept_layout(T);
  const WsLayout W = p->ws_layout(T);
  char* sv = (char*)saved;
  HIP_TRY(hipMemcpyAsync(sv + L.f[MOE_SAVED_LOGITS], logits,
                         sizeof(float) * (size_t)T * p->cfg.num_experts, hipMemcpyDeviceToDevice,
                         s));
  if (p->cfg.dtype == MOE_DTYPE_BF16) return run_routing<bf16_t>(p, s, T, sv, (char*)workspace, L, W, nullptr);
  return run_routing<float>(p, s, T, sv, (char*)workspace, L, W, nullptr);
}

const char* moe_stage_name(int32_t stage) {
  static const char* names[MOE_NUM_STAGES] = {
      "router_gemm", "route", "dispatch", "gather", "gateup_fwd", "down_fwd", "shared_fwd",
      "combine_fwd", "losses", "combine_bwd", "down_dgrad", "down_wgrad", "gateup_dgrad",
      "gateup_wgrad", "shared_bwd", "router_bwd", "dx", "recompute", "norm_fwd", "norm_bwd"};
  if (stage < 0 || stage >= MOE_NUM_STAGES) return "unknown";
  return names[stage];
}

moe_status moe_plan_set_profiling(moe_plan* p, int32_t stage_mask) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  p->profile_mask = (uint32_t)stage_mask;
  return MOE_OK;
}

moe_status moe_plan_set_shared_overlap(moe_plan* p, int32_t on) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  if (on < 0 || on > 2) return fail(MOE_ERR_INVALID, "overlap mode %d is not 0, 1 or 2", on);
  p->overlap = on;
  return MOE_OK;
}

moe_status moe_plan_stage_times(moe_plan* p, float* ms, int32_t* calls, int32_t reset) {
  moe_status st = check_plan(p);
  if (st != MOE_OK) return st;
  for (auto& q : p->pending) {
    HIP_TRY(hipEventSynchronize(q.b));
    float t = 0.0f;
    HIP_TRY(hipEventElapsedTime(&t, q.a, q.b));
    p->stage_ms[q.stage] += t;
    p->stage_calls[q.stage] += 1;
    p->free_events.push_back(q.a);
    p->free_events.push_back(q.b);
  }
  p->pending.clear();
  for (int i = 0; i < MOE_NUM_STAGES; ++i) {
    if (ms) ms[i] = p->stage_ms[i];
    if (calls) calls[i] = p->stage_calls[i];
    if (reset) {
      p->stage_ms[i] = 0.0f;
      p->stage_calls[i] = 0;
    }
  }
  return MOE_OK;
}

const char* moe_last_error(void) { return g_last_error.c_str(); }
const char* moe_version(void) { return "oxidizr-amd moe 0.1 (gfx950)"; }

}  // extern "C"
