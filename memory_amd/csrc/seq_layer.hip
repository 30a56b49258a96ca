// The sequence-routed memory layer, forward and backward, issued from one host call each.
//
// One memory layer of MemoryTransformer.forward (memory_transformer/model.py:609-692) with its
// sublayer call (memory_block.py:549-558, the caller keeps the norm and the residual):
//   pooled = mean_l h  ->  logits = pooled Wr^T + br  ->  softmax / top-k / renorm
//   (router.py:96-149)  ->  shared-chapter prepend (model.py:356-391)  ->  gather x omega ->
//   k_proj / v_proj -> attention -> o_proj (memory_attention.py:241-243, :269-478).
// The kernels are the library's own entry points (router, chapter plan, chapter GEMMs, attention,
// weight gradients); this file only orders them over three streams, so that a training step costs
// two host calls instead of one per kernel:
//
// forward   main: pool -> router linear -> top-k + prepend -> chapter plan -> K/V projection ->
//                 attention -> o_proj
//           aux:  q projection and the weight packs ([Wk; Wv], [Wk; Wv]^T, Wq^T, Wo^T), which do
//                 not depend on the routing, beside the latency-bound router launches
// backward  main: o_proj dX -> dQ (+ delta) -> dK/dV -> multi-edge sums -> K/V weight gradient
//                 -> dX of the projection into the chapters' bank rows
//           aux:  o_proj dW (beside dX / dQ); after dQ: q_proj dX (into dh, beside dK/dV); after
//                 dK/dV: the router backward and the pooling's gradient added into dh
//           fill: the dense bank gradient's zeros (beside dQ); after dQ: q_proj dW (beside dK/dV)
// Every wait is an event: the caller's stream (main) waits for aux and fill before each call
// returns, so to the caller both calls are ordinary stream-ordered work (also under graph capture).
// A wait on an event that has already completed costs nothing; one the stream reaches before the
// event completes costs ~15 us of wake-up besides the wait itself, so the side streams are given
// work that ends before the main stream reaches the join.
// Calls on one device must come from one host thread at a time (the events are per device).
#include <mutex>

#include "moc_common.h"

namespace moc {
namespace {

// Events order work on one device only, so none of them needs the system-scope release (an L2
// write-back and invalidate) a default event performs when it is recorded: a record then costs a
// stream ~3 us instead of ~4.7 us (measured with back-to-back kernels on the box).
constexpr unsigned kSeqEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;
constexpr unsigned kTimerEventFlags = hipEventDisableSystemFence;
// The K/V weight gradient runs on 192 of the 256 CUs (10 row splits per 256 x 256 tile instead of
// 14): the router backward on the aux stream then runs beside it instead of after the main
// stream's last kernel (c3: 0.936 -> 0.921 ms per step; it is ~25 us slower on its own).
constexpr int kSeqWgradBudget = 192;
constexpr int kSeqEvents = 10;  // 0..7 the schedule's, 8..9 the error-path joins (SideJoin)

struct DevEvents {
  hipEvent_t e[kSeqEvents];
  bool ready = false;
};

int seq_events(hipEvent_t** out) {
  static std::mutex mu;
  static DevEvents per_dev[64];
  int dev = 0;
  MOC_HIP(hipGetDevice(&dev));
  MOC_REQUIRE(dev >= 0 && dev < 64, MOC_ERR_UNSUPPORTED, "moc_seq_layer: device %d", dev);
  std::lock_guard<std::mutex> lock(mu);
  DevEvents& d = per_dev[dev];
  if (!d.ready) {
    for (int i = 0; i < kSeqEvents; ++i) MOC_HIP(hipEventCreateWithFlags(&d.e[i], kSeqEventFlags));
    d.ready = true;
  }
  *out = d.e;
  return MOC_OK;
}

inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// Joins the side streams a layer call has forked into the main stream on every early return (an
// error after the fork): the caller frees the layer's buffers in main-stream order once the call
// fails, so main must not run ahead of side-stream kernels that still read or write them.  The
// success path joins by the schedule's own events and disarms the guard.
struct SideJoin {
  hipStream_t main;
  hipEvent_t* ev;  // the device's event set; 8 + i joins side stream i
  hipStream_t side[2];
  int n = 0;
  void fork(hipStream_t s) { side[n++] = s; }
  void disarm() { n = 0; }
  ~SideJoin() {
    for (int i = 0; i < n; ++i) {
      if (hipEventRecord(ev[8 + i], side[i]) == hipSuccess) {
        if (hipStreamWaitEvent(main, ev[8 + i], 0) != hipSuccess) (void)hipStreamSynchronize(side[i]);
      } else {
        (void)hipStreamSynchronize(side[i]);
      }
    }
  }
};

// Optional per-stage timing (off unless armed by moc_seq_layer_timing): a timing event pair
// recorded around a stage's launches on the stream that stage runs on, so the elapsed time is
// that stage's own kernels.  One set for the process, armed on one device; used by the
// benchmark, never under graph capture.
const char* const kStageNames[] = {
    "moc_router_pool1", "moc_router_linear", "moc_router_topk_prepend", "moc_chapter_plan",
    "moc_weight_pack:wkv", "moc_rows_linear:q_proj", "moc_weight_pack:transposed", "moc_chapter_project",
    "moc_xattn_fwd", "moc_rows_linear:o_proj", "moc_linear_wgrad:o_proj", "moc_rows_linear:o_proj_dx",
    "moc_fill_zero:dbank", "moc_xattn_bwd_dq", "moc_rows_linear:q_proj_dx",
    "moc_linear_wgrad:q_proj", "moc_xattn_bwd_dkv", "moc_router_seq_bwd+linear_bwd+pool_bwd",
    "moc_dkv_multi_reduce", "moc_chapter_wgrad", "moc_chapter_dx"};
enum Stage {
  kStPool, kStRouterLinear, kStTopk, kStPlan, kStPackWkv, kStQProj, kStPackT, kStKVProj, kStAttnFwd, kStOProj,
  kStOWgrad, kStODx, kStFill, kStDq, kStQDx, kStQWgrad, kStDkv, kStRouterBwd, kStMultiReduce, kStKVWgrad,
  kStBankDx, kNumStages
};
static_assert(sizeof(kStageNames) / sizeof(kStageNames[0]) == kNumStages, "stage names");

struct StageTimer {
  uint64_t mask = 0;
  int cap = 0, dev = -1;
  hipEvent_t* ev = nullptr;  // [kNumStages][cap][2]
  int count[kNumStages] = {};
  int dropped[kNumStages] = {};
};
StageTimer g_timer;

// Records the start event of stage s on `st` and returns its pair, or nullptr when s is not armed.
hipEvent_t* stage_begin(int s, hipStream_t st) {
  StageTimer& t = g_timer;
  if (!(t.mask >> s & 1)) return nullptr;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != t.dev) return nullptr;
  if (t.count[s] >= t.cap) {
    ++t.dropped[s];
    return nullptr;
  }
  hipEvent_t* p = t.ev + ((size_t)s * t.cap + t.count[s]++) * 2;
  return hipEventRecord(p[0], st) == hipSuccess ? p : nullptr;
}

// Layout of the saved buffer (forward -> backward) and of the backward's scratch buffer.
struct SeqLayout {
  int64_t B, L, d, C;
  int H, HK, S, k, NS, KV, Lp;
  int64_t E, max_u;
  // saved
  size_t q, attn, pooled, w, uniq, n_uniq, edge_u, csr_off, csr_edge, plan_ws, wkv, wkv_t, wq_t, wo_t, kv, lse;
  size_t plan_ws_bytes, saved_bytes;
  // scratch
  size_t mlist;
  size_t d_attn, delta, dq, dkv_edge, dom_part, red, cw_ws, lw_ws, dz, dpooled, rl_ws;
  size_t cw_ws_bytes, lw_ws_bytes, rl_ws_bytes, scratch_bytes;

  int init(int64_t B_, int64_t L_, int64_t d_, int H_, int HK_, int64_t C_, int S_, int k_) {
    B = B_, L = L_, d = d_, C = C_, H = H_, HK = HK_, S = S_, k = k_;
    MOC_REQUIRE(B > 0 && B <= 64 && L > 0 && d > 0 && H > 0 && HK > 0 && H % HK == 0 && d == (int64_t)H * 64,
                MOC_ERR_UNSUPPORTED, "moc_seq_layer: B=%lld (1..64), L=%lld, d=%lld = 64 heads of 64 (H=%d, HK=%d)",
                (long long)B, (long long)L, (long long)d, H, HK);
    MOC_REQUIRE(d % 256 == 0 && (2 * HK * 64) % 256 == 0, MOC_ERR_UNSUPPORTED,
                "moc_seq_layer: d=%lld and 2*HK*64=%d must be multiples of 256", (long long)d, 2 * HK * 64);
    MOC_REQUIRE(S > 0 && S <= 1024 && k > 0 && k <= 1024 && k <= C - S && C <= 8192, MOC_ERR_UNSUPPORTED,
                "moc_seq_layer: S=%d (1..1024), k=%d (1..1024, <= C-S), C=%lld (<= 8192)", S, k, (long long)C);
    NS = S + k;
    KV = HK * 64;
    Lp = (int)((L + 127) / 128 * 128);
    E = B * NS;
    max_u = E < C ? E : C;
    const int64_t tok = B * L;
    size_t o = 0;
    auto take = [&](size_t bytes) { const size_t at = o; o = al256(o + bytes); return at; };
    q = take(tok * d * 2);
    attn = take(tok * d * 2);
    pooled = take(B * d * 4);
    w = take(B * k * 4);
    uniq = take(max_u * 4);
    n_uniq = take(2 * 4);
    edge_u = take(E * 4);
    csr_off = take((max_u + 1) * 4);
    csr_edge = take(E * 4);
    plan_ws_bytes = moc_chapter_plan_workspace(E, C);
    plan_ws = take(plan_ws_bytes);
    wkv = take((size_t)2 * KV * d * 2);
    wkv_t = take((size_t)2 * KV * d * 2);
    wq_t = take((size_t)d * d * 2);
    wo_t = take((size_t)d * d * 2);
    kv = take((size_t)max_u * 64 * 2 * KV * 2);
    lse = take((size_t)B * H * Lp * 4);
    mlist = take(dkv_multi_list_bytes(max_u));
    saved_bytes = o;
    o = 0;
    d_attn = take(tok * d * 2);
    delta = take((size_t)B * H * Lp * 4);
    dq = take(tok * d * 2);
    dkv_edge = take((size_t)E * 64 * 2 * KV * 2);
    dom_part = take((size_t)E * HK * 4);
    red = take((size_t)max_u * 64 * 2 * KV * 2);
    cw_ws_bytes = moc_chapter_wgrad_workspace(2 * KV, (int)d, max_u);
    cw_ws = take(cw_ws_bytes);
    lw_ws_bytes = moc_linear_wgrad_workspace(tok, d, d);
    lw_ws = take(lw_ws_bytes);
    dz = take((size_t)B * C * 4);
    dpooled = take((size_t)B * d * 4);
    rl_ws_bytes = moc_router_linear_bwd_workspace(B, d, C);
    rl_ws = take(rl_ws_bytes);
    scratch_bytes = o;
    return MOC_OK;
  }
};

#define SEQ_TRY(call)                  \
  do {                                 \
    if (int _rc = (call)) return _rc;  \
  } while (0)

// `call` (which may be several launches) on stream `st`, timed as stage `s` when armed
#define SEQ_STAGE(s, st, call)                                       \
  do {                                                               \
    hipEvent_t* _pair = stage_begin((s), (st));                      \
    call;                                                            \
    if (_pair) MOC_HIP(hipEventRecord(_pair[1], (st)));              \
  } while (0)

int fill_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" {

size_t moc_seq_layer_saved_bytes(int64_t B, int64_t L, int64_t d, int H, int HK, int64_t C, int S, int k) {
  SeqLayout lay;
  return lay.init(B, L, d, H, HK, C, S, k) == MOC_OK ? lay.saved_bytes : 0;
}

size_t moc_seq_layer_scratch_bytes(int64_t B, int64_t L, int64_t d, int H, int HK, int64_t C, int S, int k) {
  SeqLayout lay;
  return lay.init(B, L, d, H, HK, C, S, k) == MOC_OK ? lay.scratch_bytes : 0;
}

int moc_seq_layer_fwd(const void* h, const void* bank, const void* wr, int wr_dtype, const float* br, const void* wq,
                      const void* wk, const void* wv, const void* wo, const float* coef, int64_t B, int64_t L,
                      int64_t d, int H, int HK, int64_t C, int S, int k, float routed_scale, void* out,
                      float* logits, int32_t* idx, int32_t* idx_star, float* omega, void* saved, size_t saved_bytes,
                      hipStream_t main, hipStream_t aux) {
  MOC_REQUIRE(h && bank && wr && wq && wk && wv && wo && out && logits && idx && idx_star && omega && saved,
              MOC_ERR_ARG, "moc_seq_layer_fwd: null pointer");
  MOC_REQUIRE(main != aux, MOC_ERR_ARG, "moc_seq_layer_fwd: main and aux must be different streams");
  SeqLayout y;
  SEQ_TRY(y.init(B, L, d, H, HK, C, S, k));
  MOC_REQUIRE(saved_bytes >= y.saved_bytes, MOC_ERR_ARG, "moc_seq_layer_fwd: saved buffer %zu < %zu bytes",
              saved_bytes, y.saved_bytes);
  hipEvent_t* ev = nullptr;
  SEQ_TRY(seq_events(&ev));
  char* sv = (char*)saved;
  bf16* q = (bf16*)(sv + y.q);
  bf16* attn = (bf16*)(sv + y.attn);
  float* pooled = (float*)(sv + y.pooled);
  float* w = (float*)(sv + y.w);
  int32_t* uniq = (int32_t*)(sv + y.uniq);
  int32_t* n_uniq = (int32_t*)(sv + y.n_uniq);
  int32_t* edge_u = (int32_t*)(sv + y.edge_u);
  int32_t* csr_off = (int32_t*)(sv + y.csr_off);
  int32_t* csr_edge = (int32_t*)(sv + y.csr_edge);
  bf16* wkv = (bf16*)(sv + y.wkv);
  bf16* kv = (bf16*)(sv + y.kv);
  float* lse = (float*)(sv + y.lse);
  const int64_t tok = B * L;
  const int KV2 = 2 * y.KV;

  // aux: the [Wk; Wv] pack and the q projection beside the router (the projection's wait is on
  // them), then the transposed weights the backward reads, beside the projection and attention
  MOC_HIP(hipEventRecord(ev[0], main));
  MOC_HIP(hipStreamWaitEvent(aux, ev[0], 0));
  SideJoin join{main, ev};
  join.fork(aux);
  SEQ_STAGE(kStPackWkv, aux, SEQ_TRY(moc_weight_pack(wk, MOC_BF16, wv, MOC_BF16, y.KV, d, wkv, nullptr, aux)));
  MOC_HIP(hipEventRecord(ev[3], aux));
  SEQ_STAGE(kStQProj, aux, SEQ_TRY(moc_rows_linear(h, d, tok, wq, (int)d, (int)d, q, d, aux)));
  MOC_HIP(hipEventRecord(ev[1], aux));
  SEQ_STAGE(kStPackT, aux, {
    SEQ_TRY(moc_weight_pack(wk, MOC_BF16, wv, MOC_BF16, y.KV, d, nullptr, sv + y.wkv_t, aux));
    SEQ_TRY(moc_weight_pack(wq, MOC_BF16, (const bf16*)wq + (d / 2) * d, MOC_BF16, d / 2, d, nullptr, sv + y.wq_t,
                            aux));
    SEQ_TRY(moc_weight_pack(wo, MOC_BF16, (const bf16*)wo + (d / 2) * d, MOC_BF16, d / 2, d, nullptr, sv + y.wo_t,
                            aux));
  });

  // main: router, plan
  SEQ_STAGE(kStPool, main, SEQ_TRY(moc_router_pool1(h, MOC_BF16, B, L, d, coef, pooled, main)));
  SEQ_STAGE(kStRouterLinear, main, SEQ_TRY(moc_router_linear(pooled, B, d, wr, wr_dtype, br, C, logits, main)));
  SEQ_STAGE(kStTopk, main,
            SEQ_TRY(moc_router_topk_prepend(logits, B, C, S, k, routed_scale, idx, w, idx_star, omega, main)));
  SEQ_STAGE(kStPlan, main,
            SEQ_TRY(moc_chapter_plan(idx_star, y.E, C, sv + y.plan_ws, y.plan_ws_bytes, uniq, n_uniq, edge_u, csr_off,
                                     csr_edge, main)));
  // aux: the plan's multi-edge chapters listed for the backward's per-chapter dK|dV sums (beside
  // the projection; the list lives in the saved buffer)
  MOC_HIP(hipEventRecord(ev[4], main));
  MOC_HIP(hipStreamWaitEvent(aux, ev[4], 0));
  SEQ_TRY(dkv_multi_list(n_uniq, csr_off, csr_edge, y.max_u, (int32_t*)(sv + y.mlist), aux));
  MOC_HIP(hipEventRecord(ev[2], aux));
  // main: K/V projection (gather fused), attention, o_proj.  The projection waits for the [Wk; Wv]
  // pack only and the attention for the q projection: both events have completed when the main
  // stream reaches them, so the waits cost nothing (the q projection ends about when the router
  // does, and waiting for it before the projection cost ~6 us of wake-up).
  MOC_HIP(hipStreamWaitEvent(main, ev[3], 0));
  SEQ_STAGE(kStKVProj, main,
            SEQ_TRY(moc_chapter_project(bank, d, 1, uniq, n_uniq, y.max_u, wkv, KV2, (int)d, kv, KV2, main)));
  MOC_HIP(hipStreamWaitEvent(main, ev[1], 0));
  const int64_t span = y.max_u * 64 * KV2 - y.KV;
  SEQ_STAGE(kStAttnFwd, main,
            SEQ_TRY(moc_xattn_fwd(MOC_BF16, q, kv, kv + y.KV, span, (int64_t)64 * KV2, 64, KV2, edge_u, omega, B, L,
                                  H, HK, 64, 64, y.NS, 0.125f, attn, lse, main)));
  SEQ_STAGE(kStOProj, main, SEQ_TRY(moc_rows_linear(attn, d, tok, wo, (int)d, (int)d, out, d, main)));
  MOC_HIP(hipStreamWaitEvent(main, ev[2], 0));
  join.disarm();
  return MOC_OK;
}

int moc_seq_layer_bwd(const void* h, const void* bank, const void* wr, int wr_dtype, const float* coef, int64_t B,
                      int64_t L, int64_t d, int H, int HK, int64_t C, int S, int k, float routed_scale,
                      const float* logits, const int32_t* idx, const float* omega, const void* saved,
                      size_t saved_bytes, const void* dout, const float* dlogits, void* dh, void* dbank,
                      int64_t bank_rows, float* dwr, float* dbr, void* dwq, void* dwkv, int dwkv_dtype, void* dwo,
                      void* scratch, size_t scratch_bytes, hipStream_t main, hipStream_t aux, hipStream_t fill) {
  MOC_REQUIRE(h && bank && wr && logits && idx && omega && saved && dout && scratch, MOC_ERR_ARG,
              "moc_seq_layer_bwd: null pointer");
  MOC_REQUIRE(main != aux && main != fill && aux != fill, MOC_ERR_ARG,
              "moc_seq_layer_bwd: main, aux and fill must be three different streams");
  MOC_REQUIRE(dwkv_dtype == MOC_BF16 || dwkv_dtype == MOC_F32, MOC_ERR_UNSUPPORTED,
              "moc_seq_layer_bwd: dwkv dtype %d", dwkv_dtype);
  SeqLayout y;
  SEQ_TRY(y.init(B, L, d, H, HK, C, S, k));
  MOC_REQUIRE(saved_bytes >= y.saved_bytes && scratch_bytes >= y.scratch_bytes, MOC_ERR_ARG,
              "moc_seq_layer_bwd: saved %zu < %zu or scratch %zu < %zu bytes", saved_bytes, y.saved_bytes,
              scratch_bytes, y.scratch_bytes);
  hipEvent_t* ev = nullptr;
  SEQ_TRY(seq_events(&ev));
  const char* sv = (const char*)saved;
  const bf16* q = (const bf16*)(sv + y.q);
  const bf16* attn = (const bf16*)(sv + y.attn);
  const float* pooled = (const float*)(sv + y.pooled);
  const float* w = (const float*)(sv + y.w);
  const int32_t* uniq = (const int32_t*)(sv + y.uniq);
  const int32_t* n_uniq = (const int32_t*)(sv + y.n_uniq);
  const int32_t* edge_u = (const int32_t*)(sv + y.edge_u);
  const int32_t* csr_off = (const int32_t*)(sv + y.csr_off);
  const int32_t* csr_edge = (const int32_t*)(sv + y.csr_edge);
  const bf16* kv = (const bf16*)(sv + y.kv);
  const float* lse = (const float*)(sv + y.lse);
  char* sc = (char*)scratch;
  bf16* d_attn = (bf16*)(sc + y.d_attn);
  float* delta = (float*)(sc + y.delta);
  bf16* dq = (bf16*)(sc + y.dq);
  bf16* dkv_edge = (bf16*)(sc + y.dkv_edge);
  float* dom_part = (float*)(sc + y.dom_part);
  bf16* red = (bf16*)(sc + y.red);
  const int64_t tok = B * L;
  const int KV2 = 2 * y.KV;
  const int64_t span = y.max_u * 64 * KV2 - y.KV;
  const bool router_grads = dh || dwr || dbr;

  // aux: o_proj dW beside o_proj dX and the attention backward
  MOC_HIP(hipEventRecord(ev[0], main));
  MOC_HIP(hipStreamWaitEvent(aux, ev[0], 0));
  SideJoin join{main, ev};
  join.fork(aux);
  if (dwo)
    SEQ_STAGE(kStOWgrad, aux,
              SEQ_TRY(moc_linear_wgrad(dout, attn, MOC_BF16, tok, d, d, sc + y.lw_ws, y.lw_ws_bytes, MOC_BF16, dwo,
                                       aux)));
  MOC_HIP(hipEventRecord(ev[6], aux));  // the weight-gradient workspace is free again
  // main: o_proj dX, dQ (with the backward pre-pass's row sums delta, which dK/dV reads)
  SEQ_STAGE(kStODx, main, SEQ_TRY(moc_rows_linear(dout, d, tok, sv + y.wo_t, (int)d, (int)d, d_attn, d, main)));
  // fill: the dense bank gradient's zeros beside dQ, after o_proj's dW on the aux stream (which is
  // ordered after the caller's work, so the main stream records no event for it); started with
  // the backward, beside o_proj's dX and dW, the fill slowed o_proj's dW 55 -> 116 us and the step
  // by 25 us
  if (dbank) {
    MOC_HIP(hipStreamWaitEvent(fill, ev[6], 0));
    join.fork(fill);
    SEQ_STAGE(kStFill, fill, SEQ_TRY(moc_fill_zero(dbank, bank_rows * d * 2, fill_cus(), fill)));
    MOC_HIP(hipEventRecord(ev[2], fill));
  }
  SEQ_STAGE(kStDq, main,
            SEQ_TRY(moc_xattn_bwd_dq_delta(MOC_BF16, q, kv, kv + y.KV, span, (int64_t)64 * KV2, 64, KV2, edge_u,
                                           omega, attn, d_attn, lse, delta, B, L, H, HK, 64, 64, y.NS, 0.125f, dq,
                                           main)));
  // aux: q_proj dX into dh beside dK/dV; fill (done with the zeros by then): q_proj dW beside
  // dK/dV, so that the aux stream reaches the router backward when dK/dV ends (both on aux, they
  // ran past dK/dV's end and the router backward past the main stream's last kernel).  When
  // dK/dV is timed, its start event is the one the side streams wait on (one record, not two).
  hipEvent_t* dkv_pair = stage_begin(kStDkv, main);
  if (!dkv_pair) MOC_HIP(hipEventRecord(ev[3], main));
  const hipEvent_t after_dq = dkv_pair ? dkv_pair[0] : ev[3];
  MOC_HIP(hipStreamWaitEvent(aux, after_dq, 0));
  if (dh) SEQ_STAGE(kStQDx, aux, SEQ_TRY(moc_rows_linear(dq, d, tok, sv + y.wq_t, (int)d, (int)d, dh, d, aux)));
  if (dwq) {
    MOC_HIP(hipStreamWaitEvent(fill, after_dq, 0));
    MOC_HIP(hipStreamWaitEvent(fill, ev[6], 0));
    if (!dbank) join.fork(fill);
    SEQ_STAGE(kStQWgrad, fill,
              SEQ_TRY(moc_linear_wgrad(dq, h, MOC_BF16, tok, d, d, sc + y.lw_ws, y.lw_ws_bytes, MOC_BF16, dwq, fill)));
    MOC_HIP(hipEventRecord(ev[7], fill));
  }
  SEQ_TRY(moc_xattn_bwd_dkv(MOC_BF16, q, d_attn, kv, kv + y.KV, span, (int64_t)64 * KV2, 64, KV2, edge_u, omega, lse,
                            delta, B, L, H, HK, 64, 64, y.NS, 0.125f, dkv_edge, dom_part, main));
  // aux: the router backward from the attention's d omega and the pooling's gradient added into
  // dh, beside the K/V chapter GEMMs (on the main stream after them it measured 25 us slower);
  // when dK/dV is timed, its end event is the one the aux stream waits on
  MOC_HIP(hipEventRecord(dkv_pair ? dkv_pair[1] : ev[4], main));
  MOC_HIP(hipStreamWaitEvent(aux, dkv_pair ? dkv_pair[1] : ev[4], 0));
  if (router_grads) {
    float* dz = (float*)(sc + y.dz);
    float* dpooled = dh ? (float*)(sc + y.dpooled) : nullptr;
    SEQ_STAGE(kStRouterBwd, aux, {
      SEQ_TRY(moc_router_seq_bwd(logits, idx, w, dom_part, HK, B, C, S, k, routed_scale, dlogits, dz, aux));
      SEQ_TRY(moc_router_linear_bwd(dz, pooled, B, d, wr, wr_dtype, C, dpooled, dwr, dbr, sc + y.rl_ws,
                                    y.rl_ws_bytes, aux));
      if (dh) SEQ_TRY(moc_rows_add_bcast(dh, MOC_BF16, B, L, d, dpooled, coef, 1.f / (float)L, aux));
    });
  }
  MOC_HIP(hipEventRecord(ev[5], aux));
  // main: K/V weight gradient and the projection's dX into the bank rows
  if (dbank || dwkv)
    SEQ_STAGE(kStMultiReduce, main,
              SEQ_TRY(dkv_multi_reduce_list(dkv_edge, KV2, (const int32_t*)(sv + y.mlist), y.max_u, csr_edge, red,
                                            main)));
  if (dwkv)
    SEQ_STAGE(kStKVWgrad, main,
              SEQ_TRY(chapter_wgrad_budget(dkv_edge, KV2, red, bank, d, 1, uniq, n_uniq, y.max_u, csr_off, csr_edge,
                                           KV2, (int)d, sc + y.cw_ws, y.cw_ws_bytes, dwkv_dtype, dwkv,
                                           kSeqWgradBudget, main)));
  if (dbank) {
    // the zeros are in place before dX stores into the bank rows: the fill runs beside dQ and
    // dK/dV and has ended long before (waited for right after dQ, the step waited ~20 us for
    // it once dQ took its tiles by LDS DMA)
    MOC_HIP(hipStreamWaitEvent(main, ev[2], 0));
    SEQ_STAGE(kStBankDx, main,
              SEQ_TRY(moc_chapter_dx(dkv_edge, KV2, uniq, n_uniq, y.max_u, csr_off, csr_edge, red, sv + y.wkv_t,
                                     (int)d, KV2, MOC_BF16, dbank, d, 1, main)));
  }
  MOC_HIP(hipStreamWaitEvent(main, ev[5], 0));
  if (dwq) MOC_HIP(hipStreamWaitEvent(main, ev[7], 0));
  join.disarm();
  return MOC_OK;
}

int moc_seq_layer_stage_count(void) { return kNumStages; }

const char* moc_seq_layer_stage_name(int stage) {
  return stage >= 0 && stage < kNumStages ? kStageNames[stage] : nullptr;
}

int moc_seq_layer_timing(uint64_t stage_mask, int capacity) {
  StageTimer& t = g_timer;
  MOC_REQUIRE(capacity >= 0 && capacity <= 4096, MOC_ERR_ARG, "moc_seq_layer_timing: capacity %d (0..4096)",
              capacity);
  t.mask = 0;
  int dev = 0;
  MOC_HIP(hipGetDevice(&dev));
  if (t.ev && (t.dev != dev || (stage_mask && capacity != t.cap))) {
    for (size_t i = 0; i < (size_t)kNumStages * t.cap * 2; ++i) (void)hipEventDestroy(t.ev[i]);
    delete[] t.ev;
    t.ev = nullptr;
  }
  for (int s = 0; s < kNumStages; ++s) t.count[s] = t.dropped[s] = 0;
  if (!stage_mask || capacity == 0) return MOC_OK;
  if (!t.ev) {
    t.ev = new hipEvent_t[(size_t)kNumStages * capacity * 2];
    for (size_t i = 0; i < (size_t)kNumStages * capacity * 2; ++i)
      MOC_HIP(hipEventCreateWithFlags(&t.ev[i], kTimerEventFlags));
    t.cap = capacity;
    t.dev = dev;
  }
  t.mask = stage_mask;
  return MOC_OK;
}

int moc_seq_layer_timing_read(double* total_ms, int32_t* launches, int32_t* dropped, int n) {
  StageTimer& t = g_timer;
  MOC_REQUIRE(total_ms && launches && n >= kNumStages, MOC_ERR_ARG, "moc_seq_layer_timing_read: n=%d < %d", n,
              kNumStages);
  for (int s = 0; s < kNumStages; ++s) {
    double sum = 0.0;
    for (int i = 0; i < t.count[s]; ++i) {
      hipEvent_t* p = t.ev + ((size_t)s * t.cap + i) * 2;
      MOC_HIP(hipEventSynchronize(p[1]));
      float ms = 0.f;
      MOC_HIP(hipEventElapsedTime(&ms, p[0], p[1]));
      sum += ms;
    }
    total_ms[s] = sum;
    launches[s] = t.count[s];
    if (dropped) dropped[s] = t.dropped[s];
    t.count[s] = t.dropped[s] = 0;
  }
  return MOC_OK;
}

}  // extern "C"
