// Fused MoE layer entry points: router -> permute -> expert GEMMs ->
// shared expert -> combine, all stream-ordered on one HIP stream with no
// host synchronisation and no allocation (the caller provides the
// workspace; its size comes from the *_workspace_bytes query).
//
// Replaces ref/qwen4_exp.py:153-184 (moe_block_forward, the numpy oracle the
// serving path runs today), kernels/q4_device_decode.py:316-339 (_moe) and,
// for the DeepSeek layer, ref/deepseek_v4.py:1070-1087 (Block.moe) with the
// upstream combine of ref/hf_sources/dsv4/model.py:684-699.
//
// Two arithmetic modes:
//  prefill: activations quantized to e4m3 per 1x128 (upstream act_quant)
//           before the gate/up GEMM and again before the down GEMM; grouped
//           MFMA GEMMs over ragged row tiles.
//  decode:  fp32 activations against dequantized weights in a
//           bandwidth-bound GEMV over the touched experts only.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <mutex>

#include "../../include/sllm_moe.h"
#include "launch.h"

namespace sllm {

constexpr int PREFILL_BM = 128;
constexpr int DECODE_MAX_T = 64;
constexpr int DEC_FUSE_MAX_T = 4;  // decode batches whose gate/up finishes in-launch

struct Plan {
  bool decode;
  int N;          // T * topk
  int bm, max_tiles;
  int bm_sh;  // decode: rows per tile of the shared expert's launches
  // decode: K chunks of the streamed gate/up and down launches (routed /
  // shared) and partial-logit slices of the router GEMM
  int ks_up, ks_up_sh, ks_dn, ks_dn_sh, ks_r;
  size_t logits, w, ids, counts, offsets, sorted, inv, tiles, ntiles, pscr;
  size_t rws;  // decode: the route weight of each sorted position
  size_t xq, sx, gate, hq, hs, hq_sh, hs_sh, y, y_sh, gu, gu_sh;
  // decode, streamed kernels: item bounds of the gate/up and down launches
  // (routed and shared segments in one launch each; a DeepSeek layer whose
  // shared expert takes taller tiles than the routed experts (sh_sep) runs
  // it in launches of its own, the *_sh ones)
  long up_items, dn_items, up_sh_items, dn_sh_items;
  bool sh_sep;
  // decode, streamed kernels: stream-K deal (dec_sk_plan) of the gate/up
  // and down launches
  bool sk_up, sk_dn;
  size_t fcnt;  // decode (Qwen, T <= DEC_FUSE_MAX_T): fused finish counters,
                // then the fused combine's (fcnt_on)
  bool fcnt_on;
  size_t rpart;  // Qwen prefill router partials (RouterPart), or 0
  size_t total;
};

// Prefill: weights go through L2 (rather than streamed past it) when a
// launch's experts average more than one row tile: an expert's tiles are
// consecutive items, run at the same time on one XCD and share them
// (C4: 5.52 -> 5.33 ms). Decode launches always stream: there the tiles of
// an expert fall on different XCDs and ordinary loads only cost L2 space
// (a one-expert MLP at B=32: 150 -> 165 us).
static int weights_reused(long rows, long experts, int bm) {
  return rows > (long)bm * experts ? 1 : 0;
}

static int dense8_mode();
static bool route_inline_on();
static bool streamk_on();
static bool split_dealt_on();
static int device_cus();

static size_t take(size_t& cur, size_t bytes) {
  size_t at = cur;
  cur += align_up(bytes ? bytes : 1, 256);
  return at;
}

static bool pick_decode(int mode, int T) {
  return mode == SLLM_MOE_MODE_DECODE ||
         (mode == SLLM_MOE_MODE_AUTO && T <= DECODE_MAX_T);
}

// deepseek: the DeepSeek layer, whose shared expert's streamed projections
// are launches of their own (other weight format) rather than a second
// segment of the routed ones, and which routes every batch with the
// multi-workgroup kernels.
static Plan make_plan(int T, int H, int E, int I, int Is, int topk, int mode,
                      bool has_shared, bool need_logits, bool force_gemv,
                      bool deepseek = false) {
  Plan p{};
  p.ks_up = p.ks_up_sh = p.ks_dn = p.ks_dn_sh = 1;
  p.decode = force_gemv || pick_decode(mode, T);
  // The Qwen layer routes decode batches that fit one workgroup in one
  // fused launch (route_permute_small_fits), which would read every logit
  // slice through one CU: its router stays unsplit there. Up to
  // RI_MAX_ROUTE_T tokens the streamed layer routes inside the gate/up
  // launch instead, whose workgroups each read the slices: split there.
  const bool inl_route = !deepseek && p.decode && !force_gemv &&
                         T <= RI_MAX_ROUTE_T && route_inline_fits(T, E, topk, 0) &&
                         route_inline_on();
  const bool fused_route = !deepseek && p.decode && !inl_route &&
                           route_permute_small_fits(T, E, topk);
  p.ks_r = p.decode && need_logits && !fused_route ? router_ksplit(T, H) : 1;
  p.N = T * topk;
  if (p.decode) {
    // 16-row tiles (a touched expert's rows, mostly one tile), or 32 when
    // the experts average more than 16 rows (a dense MLP at 17-64 tokens),
    // so that each weight block is streamed once per 32 rows, not per 16
    p.bm = p.N > 16 * std::min(E, p.N) ? 32 : 16;
    p.bm_sh = deepseek ? (T > 16 ? 32 : 16) : p.bm;  // Qwen: same launches
  } else {
    p.bm = PREFILL_BM;
  }
  p.max_tiles = (int)tile_bound(p.N, E, p.bm);
  size_t c = 0;
  p.logits = need_logits ? take(c, (size_t)p.ks_r * T * E * 4) : 0;
  p.w = take(c, (size_t)p.N * 4);
  p.ids = take(c, (size_t)p.N * 4);
  p.counts = take(c, (size_t)E * 4);
  p.offsets = take(c, (size_t)(E + 1) * 4);
  p.sorted = take(c, (size_t)p.N * 4);
  p.rws = p.decode ? take(c, (size_t)p.N * 4) : 0;
  p.inv = take(c, (size_t)p.N * 4);
  p.tiles = take(c, (size_t)p.max_tiles * 16);
  p.ntiles = take(c, 4);
  p.pscr = take(c, permute_scratch_bytes(p.N, E));
  // shared-expert gate, then (split router) its ks_r partial slices
  p.gate = take(c, (size_t)(p.ks_r > 1 ? 1 + p.ks_r : 1) * T * 4);
  if (!deepseek && !p.decode && need_logits && router_topk_fits(T, E, topk, H))
    p.rpart = take(c, router_part_bytes(T, E, topk));
  if (p.decode) {
    if (!force_gemv) {  // the streamed kernels (the GEMV path does not split)
      const long rt = p.max_tiles;
      const long sh_rt = has_shared ? (T + p.bm_sh - 1) / p.bm_sh : 0;
      // DeepSeek: MXFP4 routed and FP8 shared segments share a launch (a
      // mixed-format launch) when their tiles are equally tall (up to 16
      // tokens; C4 B=1 91.5 -> 89.0 us, B=8 289 -> 278 us); taller shared
      // tiles (32 rows from 17 tokens, which stream the shared weights once
      // per 32 rows) keep launches of their own
      p.sh_sep = deepseek && has_shared && p.bm_sh != p.bm;
      if (p.sh_sep) {
        p.ks_up = dec_ksplit_up(rt * (I / 128), H / 128);
        p.ks_dn = dec_ksplit(rt * (H / 256), I / 128);
        if (has_shared) {
          p.ks_up_sh = dec_ksplit_up(sh_rt * (Is / 128), H / 128);
          p.ks_dn_sh = dec_ksplit(sh_rt * (H / 256), Is / 128);
        }
      } else if (deepseek && has_shared) {
        // mixed-format launches: an fp8 shared-expert K step streams twice
        // the bytes of an MXFP4 routed one, so the shared items count double
        // for the split and are cut twice as finely (items of equal bytes for
        // the count-based deal; gate/up only where it splits anyway, which
        // leaves the finish launch as it is)
        p.ks_up = dec_ksplit_up(rt * (I / 128) + 2 * sh_rt * (Is / 128), H / 128);
        p.ks_up_sh = p.ks_up > 1
                         ? std::min(2 * p.ks_up, std::max(1, std::min(H / 128 / 4, 8)))
                         : 1;
        p.ks_dn = dec_ksplit(rt * (H / 256) + 2 * sh_rt * (H / 256), I / 128);
        p.ks_dn_sh = std::min(2 * p.ks_dn, std::min(Is / 128, 32));
      } else {
        // the split that leaves the busiest workgroup fewest K steps under
        // the launch's row-tile chunk deal, for the tiles a uniform routing
        // touches (E (1 - (1 - 1/E)^N) experts: fewer than the bound, which
        // sizes the launch). C3 B=2 / 4 / 8 / 16: 3 / 3 / 2 / 1 slices,
        // 49.0 / 55.8 / 76.4 / 114.3 us -> 2 / 1 / 4 / 4 slices, 45.2 / 53.6 /
        // 74.0 / 110.0 us (flushed, same box, two rounds)
        // (a one-expert layer, a dense MLP, deals identity rows in eighth-
        // tile chunks: the count-based rules, as measured for it; also with
        // SLLM_MOE_SPLIT_DEALT=0)
        const int KBd = (has_shared ? std::min(I, Is) : I) / 128;
        if (E == 1 || !split_dealt_on()) {
          p.ks_up = p.ks_up_sh =
              dec_ksplit_up(rt * (I / 128) + sh_rt * (Is / 128), H / 128);
          p.ks_dn = p.ks_dn_sh =
              dec_ksplit(rt * (H / 256) + sh_rt * (H / 256), KBd);
        } else {
          const double touched = E * (1.0 - std::pow(1.0 - 1.0 / E, (double)p.N));
          const long exp_rt = std::min(
              rt, (long)std::ceil(touched + std::max(0.0, p.N - touched) / p.bm));
          const long up_upper = rt * (I / 128) + sh_rt * (Is / 128);
          p.ks_up = p.ks_up_sh = dec_ksplit_up_dealt(
              up_upper, exp_rt * (I / 128) + sh_rt * (Is / 128), I / 128,
              H / 128);
          // down: one step per item beyond its own (C3 B=2 / 3 / 7: 4 / 1 /
          // 4 -> 1 / 2 / 1 slices, 44.4 / 53.4 / 75.2 -> 43.6 / 50.3 / 74.1
          // us; other batches keep their split), for the batches the
          // gate/up rule covers; larger ones the count-based rule, which
          // keeps them unsplit (the deal-based one split C3 B=40-64 in 4
          // and its y slices took B=64 from 217 to 266 us)
          p.ks_dn = p.ks_dn_sh =
              up_upper < DEC_TARGET_ITEMS_DEALT
                  ? dec_ksplit_dealt(rt * (H / 256) + sh_rt * (H / 256),
                                     exp_rt * (H / 256) + sh_rt * (H / 256),
                                     H / 256, KBd)
                  : dec_ksplit(rt * (H / 256) + sh_rt * (H / 256), KBd);
        }
      }
      // Stream-K deal (a workgroup takes an equal range of K steps across
      // the launch's units) for the DeepSeek mixed-format launches (up to 16
      // tokens): whole items there leave a last round of a few workgroups
      // (C4 B=8 gate/up: 1040 items, the fifth round 16 items of 56 steps).
      // C4 B=1 / 2 / 4 / 8 / 16: 84.5 / 111.4 / 173.8 / 269.4 / 445.4 ->
      // 79.4 / 109.4 / 166.2 / 248.7 / 427.5 us. Elsewhere whole items stay:
      // the Qwen launches stream at the HBM rate with a fuller last round,
      // and a stream-K deal of them ran 10-25% slower per K step (C3 B=32
      // gate/up 89.5 -> 104.8 us, down 50.5 -> 57.2; workgroups' ranges
      // placed XCD-adjacent or in block order, items rotated, or units
      // permuted on the line: no better), as did the DeepSeek launches at
      // 32 and 64 tokens (651 -> 700, 898 -> 978 us).
      if (streamk_on() && deepseek && has_shared && !p.sh_sep) {
        long un[2] = {rt * (I / 128), sh_rt * (Is / 128)};
        int kb[2] = {H / 128, H / 128}, w[2] = {1, 2}, ks[2] = {1, 1};
        if (dec_sk_plan(2, un, kb, w, 8, ks)) {
          p.sk_up = true;
          p.ks_up = ks[0];
          p.ks_up_sh = ks[1];
        }
        un[0] = rt * (H / 256);
        un[1] = sh_rt * (H / 256);
        kb[0] = I / 128;
        kb[1] = Is / 128;
        if (dec_sk_plan(2, un, kb, w, 32, ks)) {
          p.sk_dn = true;
          p.ks_dn = ks[0];
          p.ks_dn_sh = ks[1];
        }
      }
      p.up_items = rt * (I / 128) * p.ks_up;
      p.dn_items = rt * (H / 256) * p.ks_dn;
      const long sh_up = sh_rt * (Is / 128) * p.ks_up_sh;
      const long sh_dn = sh_rt * (H / 256) * p.ks_dn_sh;
      if (p.sh_sep) {
        p.up_sh_items = sh_up;
        p.dn_sh_items = sh_dn;
      } else {
        p.up_items += sh_up;
        p.dn_items += sh_dn;
      }
    }
    p.hq = take(c, (size_t)p.N * I * 4);                      // h fp32
    p.hq_sh = has_shared ? take(c, (size_t)T * Is * 4) : 0;   // h_sh fp32
    p.y = take(c, (size_t)p.ks_dn * p.N * H * 4);             // y fp32 slices
    p.y_sh = has_shared ? take(c, (size_t)p.ks_dn_sh * T * H * 4) : 0;
    p.gu = p.ks_up > 1 ? take(c, (size_t)2 * p.ks_up * p.N * I * 4) : 0;
    p.gu_sh = has_shared && p.ks_up_sh > 1
                  ? take(c, (size_t)2 * p.ks_up_sh * T * Is * 4) : 0;
    // (DeepSeek: the launches that route the batch in the gate/up launch,
    // whose router launch clears the counters)
    if (!force_gemv &&
        (deepseek ? T <= RI_MAX_ROUTE_T : (T <= DEC_FUSE_MAX_T || p.sk_up))) {
      p.fcnt_on = true;
      p.fcnt = take(c, (size_t)(dec_fuse_counters(p.N, T, I, has_shared ? Is : 0) +
                                dec_combine_counters(T, H)) * 4);
    }
  } else {
    p.xq = take(c, (size_t)T * H);
    p.sx = take(c, (size_t)T * (H / 128) * 4);
    p.hq = take(c, (size_t)p.N * I);
    p.hs = take(c, (size_t)p.N * (I / 128) * 4);
    if (has_shared) {
      p.hq_sh = take(c, (size_t)T * Is);
      p.hs_sh = take(c, (size_t)T * (Is / 128) * 4);
    }
    p.y = take(c, (size_t)p.N * H * 2);                       // y bf16
    p.y_sh = has_shared ? take(c, (size_t)T * H * 2) : 0;
  }
  p.total = c;
  return p;
}

// Records the stage-boundary events when the caller asked for them.
struct StageClock {
  void** ev;
  hipStream_t st;
  mutable unsigned done = 0;  // stages whose events are recorded
  int begin(int s) const {
    if (ev) SLLM_HIP(hipEventRecord((hipEvent_t)ev[2 * s], st));
    return 0;
  }
  int end(int s) const {
    if (ev) SLLM_HIP(hipEventRecord((hipEvent_t)ev[2 * s + 1], st));
    done |= 1u << s;
    return 0;
  }
  // Stages the call did not reach: recorded with zero length at the end,
  // so that every stage's events exist on every call.
  int finish() const {
    for (int s = 0; s < SLLM_MOE_STAGES; ++s)
      if (!(done & (1u << s)) && (begin(s) || end(s))) return -1;
    return 0;
  }
};

// The code of two launch steps run in order, the second only after the
// first succeeded: the first nonzero one, so that a -2 capacity code
// reaches the entry point unchanged (an `a || b` of the two would be 1).
template <typename F, typename G>
static int first_rc(F f, G g) {
  const int rc = f();
  return rc ? rc : g();
}

// a failing stage's code (-1 error, -2 capacity) is the entry point's
#define STAGE(clk, s, call)                                                   \
  do {                                                                        \
    if ((clk).begin(s)) return -1;                                            \
    if (const int _rc = (call)) return _rc < 0 ? _rc : -1;                    \
    if ((clk).end(s)) return -1;                                              \
  } while (0)

template <typename A>
static int check_common(const A* a, const char* who) {
  SLLM_REQUIRE(a, "%s: null args", who);
  SLLM_REQUIRE(a->T > 0 && a->H > 0 && a->E > 0 && a->I > 0 && a->topk > 0,
               "%s: sizes must be positive", who);
  SLLM_REQUIRE(a->topk <= a->E && a->E <= 2048 && a->topk <= 64,
               "%s: need topk <= E <= 2048 and topk <= 64 (E=%d k=%d)", who,
               a->E, a->topk);
  SLLM_REQUIRE(a->H % 256 == 0 && a->I % 128 == 0,
               "%s: need H %% 256 == 0 and I %% 128 == 0 (H=%d I=%d)", who,
               a->H, a->I);
  SLLM_REQUIRE((long)a->T * a->topk < (1L << 30), "%s: T*topk too large", who);
  SLLM_REQUIRE(a->mode >= 0 && a->mode <= 2, "%s: bad mode %d", who, a->mode);
  SLLM_REQUIRE(a->x && a->out, "%s: null x/out", who);
  SLLM_REQUIRE(a->logits_given ? a->logits != nullptr : a->router_w != nullptr,
               "%s: need logits (logits_given) or router_w", who);
  return 0;
}

static int copy_debug(const float* logits, const float* w, const int* ids,
                      const int* counts, const int* sorted, const int* inv,
                      int T, int E, int N, float* logits_out, float* w_out,
                      int* ids_out, int* counts_out, int* sorted_out,
                      int* inv_out, hipStream_t st) {
  if (sorted_out)
    SLLM_HIP(hipMemcpyAsync(sorted_out, sorted, (size_t)N * 4,
                            hipMemcpyDeviceToDevice, st));
  if (inv_out)
    SLLM_HIP(hipMemcpyAsync(inv_out, inv, (size_t)N * 4, hipMemcpyDeviceToDevice, st));
  if (logits_out)
    SLLM_HIP(hipMemcpyAsync(logits_out, logits, (size_t)T * E * 4,
                            hipMemcpyDeviceToDevice, st));
  if (w_out)
    SLLM_HIP(hipMemcpyAsync(w_out, w, (size_t)N * 4, hipMemcpyDeviceToDevice, st));
  if (ids_out)
    SLLM_HIP(hipMemcpyAsync(ids_out, ids, (size_t)N * 4, hipMemcpyDeviceToDevice, st));
  if (counts_out)
    SLLM_HIP(hipMemcpyAsync(counts_out, counts, (size_t)E * 4,
                            hipMemcpyDeviceToDevice, st));
  return 0;
}

}  // namespace sllm

using namespace sllm;

extern "C" {

long sllm_moe_qwen_workspace_bytes(const sllm_moe_qwen_args* a) {
  if (!a || a->T <= 0 || a->E <= 0 || a->topk <= 0) {
    set_error("sllm_moe_qwen_workspace_bytes: bad args");
    return -1;
  }
  const bool sh = a->su != nullptr;
  return (long)make_plan(a->T, a->H, a->E, a->I, sh ? a->Is : 0, a->topk,
                         a->mode, sh, !a->logits_given, a->wdtype == 1)
      .total;
}

}  // extern "C"

namespace sllm {

// The Qwen layer on the workspace ws (ws_bytes bytes): the body of both
// sllm_moe_qwen_forward (caller's workspace) and
// sllm_moe_qwen_forward_noalloc (the library's per-device scratch).
static int qwen_forward_ws(const sllm_moe_qwen_args* a, char* ws,
                           long ws_bytes) {
  const bool sh = a->su != nullptr;
  SLLM_REQUIRE(a->wdtype == 0 || a->wdtype == 1,
               "sllm_moe_qwen_forward: wdtype must be 0 (fp8) or 1 (bf16)");
  const bool bf16w = a->wdtype == 1;
  SLLM_REQUIRE(a->wg && a->wu && a->wd &&
                   (bf16w || (a->wg_s && a->wu_s && a->wd_s)),
               "sllm_moe_qwen_forward: null expert weights");
  if (sh)
    SLLM_REQUIRE(a->sg && a->sd && a->sgl && a->Is > 0 && a->Is % 128 == 0 &&
                     (bf16w || (a->sg_s && a->su_s && a->sd_s)),
                 "sllm_moe_qwen_forward: incomplete shared expert");
  const int T = a->T, H = a->H, E = a->E, I = a->I, k = a->topk;
  const int Is = sh ? a->Is : 0;
  const int wf = bf16w ? 2 : 0;  // gemv weight format
  const Plan p = make_plan(T, H, E, I, Is, k, a->mode, sh, !a->logits_given,
                           bf16w);
  SLLM_REQUIRE(ws_bytes >= (long)p.total,
               "sllm_moe_qwen_forward: workspace %ld < %zu bytes", ws_bytes,
               p.total);
  hipStream_t st = (hipStream_t)a->stream;
  float* logits = a->logits_given ? (float*)a->logits : (float*)(ws + p.logits);
  float* w = (float*)(ws + p.w);
  int* ids = (int*)(ws + p.ids);
  int* counts = (int*)(ws + p.counts);
  int* offsets = (int*)(ws + p.offsets);
  int* sorted = (int*)(ws + p.sorted);
  int* inv = (int*)(ws + p.inv);
  int* tiles = (int*)(ws + p.tiles);
  int* ntiles = (int*)(ws + p.ntiles);
  float* gate = (float*)(ws + p.gate);
  const float eps = a->renorm_eps;

  const StageClock clk{a->stage_events, st};
  // One expert, top-1, logits given, streamed decode (a dense MLP run as the
  // layer): the softmax of one logit is 1 and 1 / (1 + eps) rounds to 1, so
  // every token's route weight is exactly 1 and the permutation is the
  // identity. Routing and permutation are skipped and the expert launches
  // read rows in token order (when no routing output is asked for; the
  // logits are not read, so a non-finite logit does not reach the output).
  const bool one_expert = p.decode && a->wgu_packed && E == 1 && k == 1 &&
                          a->logits_given && 1.0f + eps == 1.0f &&
                          !a->router_bias &&
                          !a->logits_out && !a->w_out && !a->ids_out &&
                          !a->counts_out && !a->sorted_out && !a->inv_pos_out;
  // Decode-size routing: the router GEMM also computes the shared-expert
  // gate, and softmax top-k runs fused with the permutation (two launches
  // instead of four). Stages a call does not run are recorded with zero
  // length, so every stage's events exist on every call.
  // Streamed decode of a routed layer at a few tokens: the gate/up launch
  // finishes its K-split items itself (DecFuse) on counters the
  // permutation launch clears, which saves the finish launch (B=1: 44 ->
  // 42 us); with the routing in the gate/up launch the router launch
  // clears them. From 5 tokens on the finish launch is as fast or faster
  // (B=8: 76.5 vs 76.9 us with the fused finish). A stream-K gate/up
  // launch (every unit in K slices) finishes in the launch at any decode
  // batch whose router launch clears the counters.
  const bool small_router = p.decode && !a->logits_given && T <= 64;
  const bool fused = p.decode && a->wgu_packed && !one_expert && !bf16w &&
                     p.fcnt_on && (p.ks_up > 1 || p.ks_up_sh > 1) &&
                     (T <= DEC_FUSE_MAX_T || (p.sk_up && small_router));
  int* fcnt = fused ? (int*)(ws + p.fcnt) : nullptr;
  const long nfcnt = fused ? dec_fuse_counters(p.N, T, I, sh ? Is : 0) : 0;
  SLLM_REQUIRE(nfcnt < (1L << 31), "sllm_moe_qwen_forward: too many counters");
  const bool small_route = p.decode && route_permute_small_fits(T, E, k);
  // Streamed decode of a routed layer: the gate/up launch builds the
  // permutation in every workgroup (the tables written out by workgroup 0)
  // in place of the permutation launch (perm_inl, after the multi-workgroup
  // routing launch), and up to 8 tokens it routes them too (route_inl, one
  // token per wave) in place of the routing launch; the router launch then
  // clears the fused finish's counters. Routing in the launch needs the
  // router launch (not the caller's logits) and leaves a split router's
  // slices unsummed (not when the caller copies the logits). Between 9 and
  // 16 tokens the one-workgroup route + permute launch is faster than
  // either (a wave's second token costs as much as the launch).
  const bool inl_ok = p.decode && a->wgu_packed && !one_expert &&
                      route_inline_fits(T, E, k, p.max_tiles) &&
                      route_inline_on();
  const bool route_inl = inl_ok && small_router && T <= RI_MAX_ROUTE_T &&
                         (!a->logits_out || p.ks_r == 1);
  // the router launch clears the fused finish's and fused combine's
  // counters when it runs; else the permutation launch clears the finish's
  const bool router_clears = small_router && p.fcnt_on && (fused || route_inl);
  const bool perm_inl = inl_ok && !route_inl && !small_route &&
                        (!fused || router_clears);
  // One token: the down launch also does the combine (DecCombine: a
  // counter per 256-column slab), which leaves three launches (router,
  // gate/up, down; B=1 39.2 -> 39.0 us). From two tokens on the units'
  // finishing queues on the last workgroups of the launch (every unit
  // completes at its end): B=2 / 4 / 8 +2.6 / +3.8 / +5.8 us, and at
  // 32-64 tokens +11-12 us, so the combine keeps its launch there.
  const bool comb_inl = route_inl && p.fcnt_on && T == 1;
  const long nccnt = comb_inl ? dec_combine_counters(T, H) : 0;
  int* ccnt = comb_inl ? (int*)(ws + p.fcnt) + dec_fuse_counters(p.N, T, I, sh ? Is : 0)
                       : nullptr;
  // the counters the router launch clears (both sets, whichever run)
  int* rzero = router_clears ? (int*)(ws + p.fcnt) : nullptr;
  const long nrzero = rzero ? dec_fuse_counters(p.N, T, I, sh ? Is : 0) + nccnt : 0;
  // Prefill: the softmax routing launch also quantizes each token's row
  // (and forms the shared-expert gate), in place of the activation-quant
  // launch (one wave per token in both; C2: 11.8 + 11.3 -> 19.8 us).
  const bool aq_fused = !p.decode && !one_expert && !small_route;
  ActQuant aq{};
  if (aq_fused) {
    aq.x = (const uint16_t*)a->x; aq.H = H; aq.pow2 = 0;
    aq.q = (uint8_t*)(ws + p.xq); aq.s = (float*)(ws + p.sx);
    aq.gate_w = sh ? (const uint16_t*)a->sgl : nullptr;
    aq.gate_out = sh ? gate : nullptr;
  }
  bool gate_done = false;
  if (one_expert) {
    STAGE(clk, SLLM_MOE_STAGE_ROUTER_GEMM, 0);
  } else if (small_router) {
    STAGE(clk, SLLM_MOE_STAGE_ROUTER_GEMM,
          launch_router_small_gate((const uint16_t*)a->x,
                                   (const uint16_t*)a->router_w, logits, T, E,
                                   H, sh ? (const uint16_t*)a->sgl : nullptr,
                                   sh ? gate : nullptr, st, p.ks_r,
                                   rzero, nrzero));
    gate_done = sh;
  }
  // split router: the routing launch finishes the gate from its partials
  float* gate_fin = small_router && sh && p.ks_r > 1 ? gate : nullptr;
  // Prefill router GEMM + softmax routing + multi-workgroup permutation: the
  // router zeroes the permutation's chunk histograms and the routing launch
  // fills them, which saves the permutation's histogram launch.
  const bool route_hist = !small_router && !one_expert && !small_route &&
                          !a->logits_given && T > 64 &&
                          permute_uses_chunk_hist(p.N, E);
  int* chunk_hist = route_hist ? (int*)(ws + p.pscr) : nullptr;
  const long hist_n =
      route_hist ? (long)((p.N + PERM_CHUNK - 1) / PERM_CHUNK) * E : 0;
  // Prefill router fused with the first half of the routing: the router
  // launch leaves each 128-expert tile's top-k and softmax partials, not
  // the (T, E) logits (written only for the caller's copy), quantizes the
  // activations and forms partial shared-expert gates from the x tiles it
  // holds; the routing launch merges the partials.
  const bool topk_router = !small_router && !one_expert && !small_route &&
                           !a->logits_given && p.rpart != 0;
  RouterPart rp{};
  if (topk_router) {
    rp = router_part_at(ws + p.rpart, T, E, k);
    rp.bias = a->router_bias;
    if (aq_fused) {
      rp.q = aq.q;
      rp.s = aq.s;
      rp.gate_w = aq.gate_w;
      rp.gate_out = aq.gate_out;
    }
  }
  if (!small_router && !one_expert) {
    STAGE(clk, SLLM_MOE_STAGE_ROUTER_GEMM,
          a->logits_given ? 0
          : topk_router
              ? launch_router_topk((const uint16_t*)a->x,
                                   (const uint16_t*)a->router_w,
                                   a->logits_out ? logits : nullptr, T, E, H,
                                   rp, st, chunk_hist, hist_n)
              : launch_router_gemm((const uint16_t*)a->x,
                                   (const uint16_t*)a->router_w, logits, T, E,
                                   H, st, 1, chunk_hist, hist_n));
  }
  if (one_expert || route_inl) {
    STAGE(clk, SLLM_MOE_STAGE_ROUTE, 0);
    STAGE(clk, SLLM_MOE_STAGE_PERMUTE, 0);
  } else if (small_route) {
    STAGE(clk, SLLM_MOE_STAGE_ROUTE,
          launch_route_permute_small(logits, w, ids, T, E, k, eps, p.bm,
                                     counts, offsets, sorted, inv, tiles,
                                     ntiles, p.max_tiles, st, p.ks_r,
                                     gate_fin, router_clears ? nullptr : fcnt,
                                     router_clears ? 0 : (int)nfcnt,
                                     a->router_bias));
    STAGE(clk, SLLM_MOE_STAGE_PERMUTE, 0);
  } else {
    STAGE(clk, SLLM_MOE_STAGE_ROUTE,
          topk_router
              ? launch_route_merge(rp, T, E, eps, w, ids, st, chunk_hist)
              : launch_route_softmax(logits, w, ids, T, E, k, eps, st, p.ks_r,
                                     gate_fin, chunk_hist,
                                     aq_fused ? &aq : nullptr,
                                     a->router_bias));
    STAGE(clk, SLLM_MOE_STAGE_PERMUTE,
          perm_inl ? 0
                   : launch_permute(ids, p.N, E, p.bm, counts, offsets, sorted,
                                    inv, tiles, ntiles, p.max_tiles,
                                    ws + p.pscr, st, route_hist,
                                    router_clears ? nullptr : fcnt,
                                    router_clears ? 0 : (int)nfcnt));
  }

  if (p.decode) {
    float* h = (float*)(ws + p.hq);
    float* y = (float*)(ws + p.y);
    STAGE(clk, SLLM_MOE_STAGE_ACT_QUANT,
          (sh && !gate_done)
              ? launch_act_quant((const uint16_t*)a->x, T, H, 0, nullptr,
                                 nullptr, (const uint16_t*)a->sgl, gate, st)
              : 0);
    float* y_sh = nullptr;
    if (a->wgu_packed) {
      // streamed packed weights (routed and shared segments in one launch
      // per projection), unquantized activations
      SLLM_REQUIRE(a->wd_packed && (!sh || (a->sgu_packed && a->sd_packed)),
                   "sllm_moe_qwen_forward: packed weights incomplete");
      float* h_sh = sh ? (float*)(ws + p.hq_sh) : nullptr;
      y_sh = sh ? (float*)(ws + p.y_sh) : nullptr;
      SegDesc r1{}, s1{};
      r1.a = (const uint8_t*)a->x; r1.sorted_idx = sorted; r1.gather = 1;
      r1.tile_info = tiles; r1.num_tiles = ntiles; r1.max_tiles = p.max_tiles;
      r1.wp = (const uint8_t*)a->wgu_packed; r1.s0 = a->wg_s; r1.s1 = a->wu_s;
      r1.N = I; r1.K = H; r1.hq = (uint8_t*)h; r1.total_rows = p.N;
      r1.ksplit = p.ks_up; r1.pp = (float*)(ws + p.gu);
      r1.pstride = (long)p.N * I;
      if (one_expert) {  // rows in token order (N = T)
        r1.sorted_idx = nullptr; r1.gather = 0;
        r1.tile_info = nullptr; r1.num_tiles = nullptr;
      }
      s1.a = (const uint8_t*)a->x; s1.total_rows = T;
      s1.wp = (const uint8_t*)a->sgu_packed; s1.s0 = a->sg_s; s1.s1 = a->su_s;
      s1.N = Is; s1.K = H; s1.hq = (uint8_t*)h_sh;
      s1.ksplit = p.ks_up_sh; s1.pp = (float*)(ws + p.gu_sh);
      s1.pstride = (long)T * Is;
      const DecFuse f_up{fcnt, (long)p.N * (I / 128)};
      RouteInline ri{};
      if (route_inl || perm_inl) {
        ri.logits = route_inl ? logits : nullptr;
        ri.ids_in = perm_inl ? ids : nullptr;
        ri.bias = a->router_bias; ri.gate = route_inl ? gate_fin : nullptr;
        ri.w = w; ri.ids = ids; ri.counts = counts; ri.offsets = offsets;
        ri.sorted = sorted; ri.inv = inv; ri.tiles = tiles; ri.ntiles = ntiles;
        ri.T = T; ri.E = E; ri.topk = k; ri.ks = p.ks_r; ri.bm = p.bm;
        ri.max_tiles = p.max_tiles; ri.eps = eps;
        ri.rw_sorted = route_inl ? (float*)(ws + p.rws) : nullptr;
      }
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
            first_rc(
                [&] {
                  return launch_stream_dec(0, 0, r1, sh ? &s1 : nullptr, k,
                                           0.f, p.up_items, st, p.bm,
                                           fused ? &f_up : nullptr,
                                           route_inl || perm_inl ? &ri : nullptr,
                                           nullptr, -1, p.sk_up);
                },
                [&] {
                  return !fused && p.ks_up > 1
                             ? launch_split_finish(r1, sh ? &s1 : nullptr,
                                                   0.f, st)
                             : 0;
                }));
      SegDesc r2{}, s2{};
      r2.a = (const uint8_t*)h; r2.sorted_idx = sorted; r2.gather = 0;
      r2.tile_info = tiles; r2.num_tiles = ntiles; r2.max_tiles = p.max_tiles;
      r2.wp = (const uint8_t*)a->wd_packed; r2.s0 = a->wd_s; r2.N = H; r2.K = I;
      r2.row_w = w; r2.row_w_by_idx = 1; r2.y = (uint16_t*)y;
      if (route_inl) {
        // workgroup 0 of the gate/up launch, which routed the batch, writes
        // the sorted positions' route weights: read by position, one load
        // rather than two dependent ones (C4 B=2 / 4: 110.2 / 168.7 ->
        // 108.5 / 166.6 us; from 17 tokens, where the weights would come
        // from the routing launch, B=32 lost 1 us)
        r2.row_w = (float*)(ws + p.rws);
        r2.row_w_by_idx = 0;
      }
      r2.ksplit = p.ks_dn; r2.pstride = (long)p.N * H;
      if (one_expert) {  // route weights are exactly 1
        r2.total_rows = p.N;
        r2.sorted_idx = nullptr; r2.tile_info = nullptr; r2.num_tiles = nullptr;
        r2.row_w = nullptr; r2.row_w_by_idx = 0;
      }
      s2.a = (const uint8_t*)h_sh; s2.total_rows = T;
      s2.wp = (const uint8_t*)a->sd_packed; s2.s0 = a->sd_s; s2.N = H;
      s2.K = Is; s2.row_w = gate; s2.y = (uint16_t*)y_sh;
      s2.ksplit = p.ks_dn_sh; s2.pstride = (long)T * H;
      DecCombine dc{};
      if (comb_inl) {
        dc.cnt = ccnt; dc.inv = inv; dc.sorted = sorted;
        dc.y = y; dc.kstride = (long)p.N * H; dc.ks = p.ks_dn;
        dc.y_sh = sh ? y_sh : nullptr; dc.kstride_sh = (long)T * H;
        dc.ks_sh = sh ? p.ks_dn_sh : 0;
        dc.T = T; dc.H = H; dc.topk = k; dc.out_f32 = a->out_f32;
        dc.out = a->out;
      }
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
            launch_stream_dec(0, 1, r2, sh ? &s2 : nullptr, k, 0.f,
                              p.dn_items, st, p.bm, nullptr, nullptr,
                              comb_inl ? &dc : nullptr, -1, p.sk_dn));
      STAGE(clk, SLLM_MOE_STAGE_SHARED_UP, 0);
      STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN, 0);
      STAGE(clk, SLLM_MOE_STAGE_COMBINE,
            comb_inl ? 0
                     : launch_combine_split(y, one_expert ? nullptr : inv, k,
                                            y_sh, T, H, a->out_f32, a->out,
                                            p.ks_dn, (long)p.N * H, p.ks_dn_sh,
                                            (long)T * H, st));
    } else {
    STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
          launch_gemv(wf, 1, a->x, 1, 1, sorted, k, p.N, tiles, ntiles,
          p.max_tiles, offsets, (const uint8_t*)a->wg, a->wg_s,
          (const uint8_t*)a->wu, a->wu_s, I, H, nullptr, 0.f, h, st));
    STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
          launch_gemv(wf, 0, h, 0, 0, sorted, k, p.N, tiles, ntiles, p.max_tiles,
          offsets, (const uint8_t*)a->wd, a->wd_s, nullptr, nullptr,
          H, I, w, 0.f, y, st));
    if (sh) {
      float* h_sh = (float*)(ws + p.hq_sh);
      y_sh = (float*)(ws + p.y_sh);
      STAGE(clk, SLLM_MOE_STAGE_SHARED_UP,
            launch_gemv(wf, 1, a->x, 1, 0, nullptr, k, T, nullptr, nullptr, 1,
            nullptr, (const uint8_t*)a->sg, a->sg_s,
            (const uint8_t*)a->su, a->su_s, Is, H, nullptr, 0.f,
            h_sh, st));
      STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN,
            launch_gemv(wf, 0, h_sh, 0, 0, nullptr, k, T, nullptr, nullptr, 1,
            nullptr, (const uint8_t*)a->sd, a->sd_s, nullptr,
            nullptr, H, Is, gate, 0.f, y_sh, st));
    }
    STAGE(clk, SLLM_MOE_STAGE_COMBINE,
          launch_combine(y, 1, inv, k, y_sh, T, H, a->out_f32, a->out, st));
    }
  } else {
    uint8_t* xq = (uint8_t*)(ws + p.xq);
    float* sx = (float*)(ws + p.sx);
    uint8_t* hq = (uint8_t*)(ws + p.hq);
    float* hs = (float*)(ws + p.hs);
    uint16_t* y = (uint16_t*)(ws + p.y);
    STAGE(clk, SLLM_MOE_STAGE_ACT_QUANT,
          aq_fused ? 0
                   : launch_act_quant((const uint16_t*)a->x, T, H, 0, xq, sx,
                                      sh ? (const uint16_t*)a->sgl : nullptr,
                                      gate, st));
    uint16_t* y_sh = nullptr;
    uint8_t* hq_sh = nullptr;
    float* hs_sh = nullptr;
    if (sh) {
      hq_sh = (uint8_t*)(ws + p.hq_sh);
      hs_sh = (float*)(ws + p.hs_sh);
      y_sh = (uint16_t*)(ws + p.y_sh);
    }
    if (a->wgu_packed) {
      SLLM_REQUIRE(a->wd_packed && (!sh || (a->sgu_packed && a->sd_packed)),
                   "sllm_moe_qwen_forward: packed weights incomplete");
      const long sh_rt = sh ? (T + 127) / 128 : 0;
      SegDesc r1{}, s1{};
      r1.wreuse = weights_reused(p.N, E, PREFILL_BM);
      r1.a = xq; r1.sa = sx; r1.sorted_idx = sorted; r1.gather = 1;
      r1.tile_info = tiles; r1.num_tiles = ntiles; r1.max_tiles = p.max_tiles;
      r1.wp = (const uint8_t*)a->wgu_packed; r1.s0 = a->wg_s; r1.s1 = a->wu_s;
      r1.N = I; r1.K = H; r1.hq = hq; r1.hs = hs;
      s1.a = xq; s1.sa = sx; s1.total_rows = T;
      s1.wp = (const uint8_t*)a->sgu_packed; s1.s0 = a->sg_s; s1.s1 = a->su_s;
      s1.N = Is; s1.K = H; s1.hq = hq_sh; s1.hs = hs_sh;
      const long up1 = (long)p.max_tiles * (I / 128) + sh_rt * (Is / 128);
      // SLLM_MOE_DENSE8=2 with experts averaging more than one row tile:
      // the compute-dense FP8 kernel, one launch per segment (the shared
      // expert's too once its rows fill more than one tile).
      const bool rdense = dense8_mode() == 2 && r1.wreuse;
      const bool sdense = rdense && sh && T > PREFILL_BM;
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
            rdense && dense8_fits(0, r1)
                ? first_rc(
                      [&] {
                        return launch_dense8(0, r1, 1, k, 0.f, 0, st,
                                             device_cus());
                      },
                      [&] {
                        return !sh ? 0
                               : sdense && dense8_fits(0, s1)
                                   ? launch_dense8(0, s1, 1, k, 0.f, 0, st,
                                                   device_cus())
                                   : launch_stream(0, 0, s1, nullptr, k, 0.f, 0,
                                                   sh_rt * (Is / 128), st);
                      })
                : launch_stream(0, 0, r1, sh ? &s1 : nullptr, k, 0.f, 0, up1, st));
      SegDesc r2{}, s2{};
      r2.wreuse = weights_reused(p.N, E, PREFILL_BM);
      r2.a = hq; r2.sa = hs; r2.sorted_idx = sorted; r2.gather = 0;
      r2.tile_info = tiles; r2.num_tiles = ntiles; r2.max_tiles = p.max_tiles;
      r2.wp = (const uint8_t*)a->wd_packed; r2.s0 = a->wd_s; r2.N = H; r2.K = I;
      r2.row_w = w; r2.row_w_by_idx = 1; r2.y = y;
      s2.a = hq_sh; s2.sa = hs_sh; s2.total_rows = T;
      s2.wp = (const uint8_t*)a->sd_packed; s2.s0 = a->sd_s; s2.N = H;
      s2.K = Is; s2.row_w = gate; s2.y = y_sh;
      const long up2 = (long)p.max_tiles * (H / 256) + sh_rt * (H / 256);
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
            rdense && dense8_fits(1, r2)
                ? first_rc(
                      [&] {
                        return launch_dense8(1, r2, 1, k, 0.f, 0, st,
                                             device_cus());
                      },
                      [&] {
                        return !sh ? 0
                               : sdense && dense8_fits(1, s2)
                                   ? launch_dense8(1, s2, 1, k, 0.f, 0, st,
                                                   device_cus())
                                   : launch_stream(0, 1, s2, nullptr, k, 0.f, 0,
                                                   sh_rt * (H / 256), st);
                      })
                : launch_stream(0, 1, r2, sh ? &s2 : nullptr, k, 0.f, 0, up2, st));
      // the shared expert ran inside the two launches above
      STAGE(clk, SLLM_MOE_STAGE_SHARED_UP, 0);
      STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN, 0);
    } else {
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
            launch_gemm1_fp8(xq, sx, sorted, k, p.N, tiles, ntiles,
                             p.max_tiles, offsets, (const uint8_t*)a->wg,
                             a->wg_s, (const uint8_t*)a->wu, a->wu_s, I, H,
                             nullptr, 0.f, 0, hq, hs, st));
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
            launch_gemm2_fp8(hq, hs, sorted, k, p.N, tiles, ntiles,
                             p.max_tiles, offsets, (const uint8_t*)a->wd,
                             a->wd_s, I, H, w, y, st));
      if (sh) {
        STAGE(clk, SLLM_MOE_STAGE_SHARED_UP,
              launch_gemm1_fp8(xq, sx, nullptr, k, T, nullptr, nullptr, 0,
                               nullptr, (const uint8_t*)a->sg, a->sg_s,
                               (const uint8_t*)a->su, a->su_s, Is, H, nullptr,
                               0.f, 0, hq_sh, hs_sh, st));
        STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN,
              launch_gemm2_fp8(hq_sh, hs_sh, nullptr, k, T, nullptr, nullptr,
                               0, nullptr, (const uint8_t*)a->sd, a->sd_s, Is,
                               H, gate, y_sh, st));
      }
    }
    STAGE(clk, SLLM_MOE_STAGE_COMBINE,
          launch_combine(y, 0, inv, k, y_sh, T, H, a->out_f32, a->out, st));
  }
  if (clk.finish()) return -1;
  return copy_debug(logits, w, ids, counts, sorted, inv, T, E, p.N,
                    a->logits_out, a->w_out, a->ids_out, a->counts_out,
                    a->sorted_out, a->inv_pos_out, st);
}

// ---------------------------------------------------------------------------
// Workspace of the no-allocation entry point: one array per device (each
// device's code object holds its own copy at its own address), kept until
// the process ends. Its device address comes from hipGetSymbolAddress, once
// per device, with that device current; host code uses only that address
// (the array's name is a host-side stand-in). Calls that overlap on one
// device share (and race on) it. The layer writes every workspace word it
// reads within the call, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
constexpr long SCRATCH_BYTES = 32L << 20;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
static std::once_flag scratch_once[SCRATCH_MAX_DEVICES];
static void* scratch_addr[SCRATCH_MAX_DEVICES];
static hipError_t scratch_rc[SCRATCH_MAX_DEVICES];

static int scratch_of_current_device(char** out) {
  int dev = -1;
  SLLM_HIP(hipGetDevice(&dev));
  SLLM_REQUIRE(dev >= 0 && dev < SCRATCH_MAX_DEVICES,
               "no-alloc layer: device %d beyond %d", dev, SCRATCH_MAX_DEVICES);
  std::call_once(scratch_once[dev], [dev] {
    void* ptr = nullptr;
    scratch_rc[dev] = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    scratch_addr[dev] = ptr;
  });
  SLLM_REQUIRE(scratch_rc[dev] == hipSuccess && scratch_addr[dev] != nullptr,
               "no-alloc layer: hipGetSymbolAddress(scratch) on device %d: %s",
               dev, hipGetErrorString(scratch_rc[dev]));
  *out = (char*)scratch_addr[dev];
  return 0;
}

}  // namespace sllm

extern "C" {

int sllm_moe_qwen_forward(const sllm_moe_qwen_args* a) {
  if (check_common(a, "sllm_moe_qwen_forward")) return -1;
  SLLM_REQUIRE(a->workspace, "sllm_moe_qwen_forward: null workspace");
  return qwen_forward_ws(a, (char*)a->workspace, a->workspace_bytes);
}

// ---- graphs of one layer call (decode loops: fixed buffers, many calls) ----
struct LayerGraph {
  hipGraph_t graph;
  hipGraphExec_t exec;
};

void* sllm_moe_qwen_graph_new(const sllm_moe_qwen_args* a) {
  if (check_common(a, "sllm_moe_qwen_graph_new")) return nullptr;
  if (a->stage_events) {
    set_error("sllm_moe_qwen_graph_new: stage events cannot be captured");
    return nullptr;
  }
  hipStream_t cs = nullptr;
  if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) {
    set_error("sllm_moe_qwen_graph_new: hipStreamCreateWithFlags failed");
    return nullptr;
  }
  sllm_moe_qwen_args c = *a;
  c.stream = cs;
  LayerGraph* g = new LayerGraph{nullptr, nullptr};
  int rc = 0;
  hipError_t e = hipStreamBeginCapture(cs, hipStreamCaptureModeRelaxed);
  if (e == hipSuccess) {
    rc = sllm_moe_qwen_forward(&c);
    hipError_t e2 = hipStreamEndCapture(cs, &g->graph);  // ends it on error too
    if (rc == 0 && e2 != hipSuccess) {
      set_error("sllm_moe_qwen_graph_new: hipStreamEndCapture: %s",
                hipGetErrorString(e2));
      rc = -1;
    }
    if (rc == 0 && hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0) !=
                       hipSuccess) {
      set_error("sllm_moe_qwen_graph_new: hipGraphInstantiate failed");
      rc = -1;
    }
  } else {
    set_error("sllm_moe_qwen_graph_new: hipStreamBeginCapture: %s",
              hipGetErrorString(e));
    rc = -1;
  }
  (void)hipStreamDestroy(cs);
  if (rc) {
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return nullptr;
  }
  return g;
}

int sllm_moe_graph_launch(void* graph, void* stream) {
  SLLM_REQUIRE(graph, "sllm_moe_graph_launch: null graph");
  SLLM_HIP(hipGraphLaunch(((LayerGraph*)graph)->exec, (hipStream_t)stream));
  return 0;
}

int sllm_moe_graph_free(void* graph) {
  if (!graph) return 0;
  LayerGraph* g = (LayerGraph*)graph;
  const hipError_t e1 = hipGraphExecDestroy(g->exec);
  const hipError_t e2 = hipGraphDestroy(g->graph);
  delete g;
  SLLM_REQUIRE(e1 == hipSuccess && e2 == hipSuccess, "sllm_moe_graph_free failed");
  return 0;
}

long sllm_moe_qwen_forward_noalloc_max_bytes(void) { return SCRATCH_BYTES; }

int sllm_moe_qwen_forward_noalloc(const sllm_moe_qwen_args* a) {
  if (check_common(a, "sllm_moe_qwen_forward_noalloc")) return -1;
  SLLM_REQUIRE(!a->workspace && a->workspace_bytes == 0,
               "sllm_moe_qwen_forward_noalloc: pass no workspace (the "
               "library's per-device scratch is used)");
  const long need = sllm_moe_qwen_workspace_bytes(a);
  if (need < 0) return -1;
  SLLM_CAPACITY(need <= SCRATCH_BYTES,
                "sllm_moe_qwen_forward_noalloc: this call needs %ld workspace "
                "bytes, above the %ld-byte scratch (T=%d H=%d E=%d I=%d k=%d "
                "mode %d); use sllm_moe_qwen_forward with a workspace",
                need, SCRATCH_BYTES, a->T, a->H, a->E, a->I, a->topk, a->mode);
  char* ws = nullptr;
  if (scratch_of_current_device(&ws)) return -1;
  return qwen_forward_ws(a, ws, SCRATCH_BYTES);
}

long sllm_moe_ds_workspace_bytes(const sllm_moe_ds_args* a) {
  if (!a || a->T <= 0 || a->E <= 0 || a->topk <= 0) {
    set_error("sllm_moe_ds_workspace_bytes: bad args");
    return -1;
  }
  const bool sh = a->s1 != nullptr;
  return (long)make_plan(a->T, a->H, a->E, a->I, sh ? a->Is : 0, a->topk,
                         a->mode, sh, !a->logits_given, false, true)
      .total;
}

// Host plan query (no device work): the tiling and K splits the layer picks
// for a shape, and for each streamed decode launch (gate/up, down, and the
// DeepSeek shared expert's two) its item bound, XCD deal chunk and grid.
int sllm_moe_plan_query(int deepseek, int T, int H, int E, int I, int Is,
                        int topk, int mode, int logits_given, long* out,
                        int n_out) {
  SLLM_REQUIRE(out && n_out >= SLLM_MOE_PLAN_FIELDS && T > 0 && H > 0 &&
                   E > 0 && I > 0 && Is >= 0 && topk > 0 && topk <= E &&
                   H % 256 == 0 && I % 128 == 0 && Is % 128 == 0 &&
                   mode >= 0 && mode <= 2,
               "sllm_moe_plan_query: bad args (T=%d H=%d E=%d I=%d Is=%d "
               "k=%d mode %d, %d outputs)", T, H, E, I, Is, topk, mode, n_out);
  const Plan p = make_plan(T, H, E, I, Is, topk, mode, Is > 0, !logits_given,
                           false, deepseek != 0);
  for (int i = 0; i < SLLM_MOE_PLAN_FIELDS; ++i) out[i] = 0;
  out[0] = p.decode;
  out[1] = p.bm;
  out[2] = p.bm_sh;
  out[3] = p.max_tiles;
  out[4] = p.ks_r;
  out[5] = p.ks_up;
  out[6] = p.ks_up_sh;
  out[7] = p.ks_dn;
  out[8] = p.ks_dn_sh;
  out[9] = device_cus();
  if (!p.decode) return 0;
  // the first segment of each launch decides its deal chunk
  const int segN[4] = {I, H, Is, H}, ntw[4] = {128, 256, 128, 256};
  const int segks[4] = {p.ks_up, p.ks_dn, p.ks_up_sh, p.ks_dn_sh};
  const long items[4] = {p.up_items, p.dn_items, p.up_sh_items, p.dn_sh_items};
  const bool sk[4] = {p.sk_up, p.sk_dn, false, false};
  const long sh_rt = Is > 0 ? (T + p.bm_sh - 1) / p.bm_sh : 0;
  const bool two = Is > 0 && !p.sh_sep;  // shared segment in launches 0, 1
  for (int j = 0; j < 4; ++j) {
    if (items[j] <= 0) continue;
    out[10 + 3 * j] = items[j];
    if (sk[j]) {  // stream-K (routed + shared launches): chunk 0, the grid
                  // from the cost line's bound
      const bool up = j == 0;
      const long un[2] = {(long)p.max_tiles * (up ? I / 128 : H / 256),
                          sh_rt * (up ? Is / 128 : H / 256)};
      const int kb[2] = {up ? H / 128 : I / 128, up ? H / 128 : Is / 128};
      const int w[2] = {1, deepseek ? 2 : 1};
      const int ks[2] = {up ? p.ks_up : p.ks_dn, up ? p.ks_up_sh : p.ks_dn_sh};
      out[11 + 3 * j] = 0;
      out[12 + 3 * j] = dec_sk_launch_grid(two ? 2 : 1, un, kb, w, ks);
      continue;
    }
    // the routed launches' rows come from the tile table (identity rows for
    // a one-expert Qwen layer, run as a dense MLP), the DeepSeek shared
    // expert's are identity rows
    const bool routed = j < 2 && (deepseek || E > 1 || topk > 1);
    const long cb = dec_deal_chunk(segN[j], ntw[j], segks[j], routed, items[j]);
    out[11 + 3 * j] = cb;
    out[12 + 3 * j] = dec_launch_grid(items[j], cb);
  }
  return 0;
}

}  // extern "C"

namespace sllm {

static int device_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

// The DeepSeek layer's routed projections run on the compute-dense kernel
// in prefill over packed MXFP4 weights when the experts average more than
// one 128-row tile. SLLM_MOE_DENSE=0 in the environment keeps the
// streaming kernel (same arithmetic, for comparisons).
// The compute-dense FP8 kernel (gemm_dense8.hip) where it measured faster:
// the DeepSeek shared expert's gate/up at more than one row tile (C4:
// 327 -> 287 us). Slower where not used: that expert's down projection
// (174 -> 178 us) and the skewed Qwen layer's routed projections (C5
// gate/up 541 -> 593 us, down 379 -> 521 us: its 256-column items, all
// that three LDS stages hold with fp8 weights, leave the per-step barrier
// and load issue larger than the step's MFMAs). SLLM_MOE_DENSE8=0 keeps
// every FP8 projection on the streaming kernel, =2 runs it wherever it
// fits (both give the same bits).
static int dense8_mode() {
  const char* v = std::getenv("SLLM_MOE_DENSE8");
  return v && v[0] == '0' ? 0 : (v && v[0] == '2' ? 2 : 1);
}

// SLLM_MOE_ROUTE_INLINE=0: decode routes in its own launches (the same
// tables, bit for bit).
// SLLM_MOE_STREAMK=0: decode launches deal whole (K-split) items instead
// of stream-K ranges (A/B runs)
static bool streamk_on() {
  const char* v = std::getenv("SLLM_MOE_STREAMK");
  return !(v && v[0] == '0');
}

static bool split_dealt_on() {
  const char* v = std::getenv("SLLM_MOE_SPLIT_DEALT");
  return !(v && v[0] == '0');
}

static bool route_inline_on() {
  const char* v = std::getenv("SLLM_MOE_ROUTE_INLINE");
  return !(v && v[0] == '0');
}

static bool dense_layer(const sllm_moe_ds_args* a) {
  const char* env = getenv("SLLM_MOE_DENSE");
  if (env && env[0] == '0') return false;
  return a->w13_packed && !pick_decode(a->mode, a->T) &&
         (long)a->T * a->topk > (long)PREFILL_BM * a->E && a->I % 256 == 0 &&
         a->H % 512 == 0;
}

}  // namespace sllm

extern "C" {

int sllm_moe_ds_forward(const sllm_moe_ds_args* a) {
  if (check_common(a, "sllm_moe_ds_forward")) return -1;
  SLLM_REQUIRE(a->workspace, "sllm_moe_ds_forward: null workspace");
  SLLM_REQUIRE(!a->tid2eid || (a->token_ids && a->vocab > 0),
               "sllm_moe_ds_forward: hash routing needs token_ids and vocab");
  const bool sh = a->s1 != nullptr;
  SLLM_REQUIRE(a->w1 && a->w1_s && a->w3 && a->w3_s && a->w2 && a->w2_s,
               "sllm_moe_ds_forward: null expert weights");
  SLLM_REQUIRE(a->H % 32 == 0 && a->I % 32 == 0, "sllm_moe_ds_forward: H, I");
  if (sh)
    SLLM_REQUIRE(a->s1_s && a->s3 && a->s3_s && a->s2 && a->s2_s && a->Is > 0 &&
                     a->Is % 128 == 0,
                 "sllm_moe_ds_forward: incomplete shared expert");
  const int T = a->T, H = a->H, E = a->E, I = a->I, k = a->topk;
  const int Is = sh ? a->Is : 0;
  const float L = a->swiglu_limit;
  const bool dense = dense_layer(a);
  const Plan p = make_plan(T, H, E, I, Is, k, a->mode, sh, !a->logits_given,
                           false, true);
  SLLM_REQUIRE(a->workspace_bytes >= (long)p.total,
               "sllm_moe_ds_forward: workspace %ld < %zu bytes",
               a->workspace_bytes, p.total);
  hipStream_t st = (hipStream_t)a->stream;
  char* ws = (char*)a->workspace;
  float* logits = a->logits_given ? (float*)a->logits : (float*)(ws + p.logits);
  float* w = (float*)(ws + p.w);
  int* ids = (int*)(ws + p.ids);
  int* counts = (int*)(ws + p.counts);
  int* offsets = (int*)(ws + p.offsets);
  int* sorted = (int*)(ws + p.sorted);
  int* inv = (int*)(ws + p.inv);
  int* tiles = (int*)(ws + p.tiles);
  int* ntiles = (int*)(ws + p.ntiles);

  const StageClock clk{a->stage_events, st};
  // Prefill: the router launch also quantizes the activations (power-of-two
  // scales) from the x chunks it stages, in place of the activation-quant
  // launch, which would read x again (C4: 117 MB).
  const bool rq_fused = !p.decode && !a->logits_given &&
                        router_logits_quant_fits(T, H);
  // Streamed decode up to RI_MAX_ROUTE_T tokens with the router launch: the
  // routed gate/up launch also routes the batch (grouped scoring, a token
  // per wave, in every workgroup), in place of the routing launch; the
  // router launch clears the counters of the gate/up launch's fused finish
  // and, at one token, of the down launch's fused combine (as in the Qwen
  // layer). Not with hash routing, caller-given logits, or a split
  // router's logits asked for (the launch leaves the slices unsummed).
  const bool route_inl = p.decode && a->w13_packed && p.fcnt_on &&
                         !a->tid2eid && !a->logits_given &&
                         T <= RI_MAX_ROUTE_T && E <= RI_MAX_E_GROUPED &&
                         (!a->logits_out || p.ks_r == 1) &&
                         route_inline_fits(T, E, k, p.max_tiles) &&
                         route_inline_on();
  const bool fused = route_inl && (p.ks_up > 1 || (sh && p.ks_up_sh > 1));
  // (the down launch's fused combine, a gain for the Qwen layer at one
  // token, lost here: C4 B=1 down 24.2 -> 31.6 us against the 4.3 us
  // combine launch, with H / 256 = 28 units of 8 routed K-split slots and
  // the shared slices to add at the launch's end)
  const bool comb_inl = false;
  int* fcnt = route_inl ? (int*)(ws + p.fcnt) : nullptr;
  const long nfcnt = route_inl ? dec_fuse_counters(p.N, T, I, Is) : 0;
  const long nccnt = comb_inl ? dec_combine_counters(T, H) : 0;
  // with caller-provided logits the router stage is recorded with zero
  // length, so every stage's events exist on every call
  STAGE(clk, SLLM_MOE_STAGE_ROUTER_GEMM,
        a->logits_given ? 0
        : rq_fused
            ? launch_router_logits_quant(
                  (const uint16_t*)a->x, (const uint16_t*)a->router_w, logits,
                  T, E, H, (uint8_t*)(ws + p.xq), (float*)(ws + p.sx), 1, st)
        : route_inl
            ? launch_router_small_gate((const uint16_t*)a->x,
                                       (const uint16_t*)a->router_w, logits,
                                       T, E, H, nullptr, nullptr, st, p.ks_r,
                                       fcnt, nfcnt + nccnt)
            : launch_router_gemm((const uint16_t*)a->x,
                                 (const uint16_t*)a->router_w, logits, T, E,
                                 H, st, p.ks_r));
  STAGE(clk, SLLM_MOE_STAGE_ROUTE,
        route_inl ? 0
        : a->tid2eid
            ? launch_route_hash(logits, a->token_ids, a->tid2eid, a->vocab, w,
                                ids, T, E, k, a->scoring, a->route_scale, st,
                                p.ks_r)
            : launch_route_grouped(logits, a->bias, w, ids, T, E, k,
                                   a->n_group, a->topk_group, a->scoring,
                                   a->route_scale, st, p.ks_r));
  // Streamed decode otherwise: the routed gate/up launch builds the
  // permutation from the routing launch's ids in every workgroup
  // (RouteInline.ids_in), in place of the permutation launch, as in the
  // Qwen layer.
  const bool perm_inl = p.decode && a->w13_packed && !route_inl &&
                        route_inline_fits(T, E, k, p.max_tiles) &&
                        route_inline_on();
  STAGE(clk, SLLM_MOE_STAGE_PERMUTE,
        route_inl || perm_inl
            ? 0
            : launch_permute(ids, p.N, E, p.bm, counts, offsets, sorted, inv,
                             tiles, ntiles, p.max_tiles, ws + p.pscr, st));

  if (p.decode && a->w13_packed) {
    // streamed packed weights, unquantized activations; the route weight
    // scales the down projection's rows as in the GEMV decode below
    SLLM_REQUIRE(a->w13_s_packed && a->w2_packed && a->w2_s_packed &&
                     (!sh || (a->s13_packed && a->s2_packed)),
                 "sllm_moe_ds_forward: packed weights incomplete");
    float* h = (float*)(ws + p.hq);
    float* y = (float*)(ws + p.y);
    float* h_sh = sh ? (float*)(ws + p.hq_sh) : nullptr;
    float* y_sh = sh ? (float*)(ws + p.y_sh) : nullptr;
    // shared expert (fp8, identity rows): the second segment of the routed
    // launches (a mixed-format launch), or launches of its own (sh_sep)
    SegDesc s1{};
    s1.a = (const uint8_t*)a->x; s1.total_rows = T;
    s1.wp = (const uint8_t*)a->s13_packed; s1.s0 = a->s1_s; s1.s1 = a->s3_s;
    s1.N = Is; s1.K = H; s1.hq = (uint8_t*)h_sh;
    s1.ksplit = p.ks_up_sh; s1.pp = (float*)(ws + p.gu_sh);
    s1.pstride = (long)T * Is;
    SegDesc s2{};
    s2.a = (const uint8_t*)h_sh; s2.total_rows = T;
    s2.wp = (const uint8_t*)a->s2_packed; s2.s0 = a->s2_s;
    s2.N = H; s2.K = Is; s2.y = (uint16_t*)y_sh;
    s2.ksplit = p.ks_dn_sh; s2.pstride = (long)T * H;
    const bool sh_in = sh && !p.sh_sep;
    SegDesc r1{};
    r1.a = (const uint8_t*)a->x; r1.sorted_idx = sorted; r1.gather = 1;
    r1.tile_info = tiles; r1.num_tiles = ntiles; r1.max_tiles = p.max_tiles;
    r1.wp = (const uint8_t*)a->w13_packed; r1.s0 = a->w13_s_packed;
    r1.N = I; r1.K = H; r1.hq = (uint8_t*)h; r1.total_rows = p.N;
    r1.ksplit = p.ks_up; r1.pp = (float*)(ws + p.gu);
    r1.pstride = (long)p.N * I;
    SegDesc r2{};
    r2.a = (const uint8_t*)h; r2.sorted_idx = sorted; r2.gather = 0;
    r2.tile_info = tiles; r2.num_tiles = ntiles; r2.max_tiles = p.max_tiles;
    r2.wp = (const uint8_t*)a->w2_packed; r2.s0 = a->w2_s_packed;
    r2.N = H; r2.K = I; r2.row_w = w; r2.row_w_by_idx = 1; r2.y = (uint16_t*)y;
    r2.ksplit = p.ks_dn; r2.pstride = (long)p.N * H;
    RouteInline ri{};
    if (route_inl || perm_inl) {
      ri.logits = route_inl ? logits : nullptr;
      ri.ids_in = perm_inl ? ids : nullptr;
      ri.bias = a->bias; ri.w = w; ri.ids = ids;
      ri.counts = counts; ri.offsets = offsets; ri.sorted = sorted;
      ri.inv = inv; ri.tiles = tiles; ri.ntiles = ntiles;
      ri.T = T; ri.E = E; ri.topk = k; ri.ks = route_inl ? p.ks_r : 1;
      ri.bm = p.bm; ri.max_tiles = p.max_tiles;
      ri.grouped = route_inl; ri.scoring = a->scoring; ri.n_group = a->n_group;
      ri.topk_group = a->topk_group; ri.route_scale = a->route_scale;
      // routed here: workgroup 0 writes the sorted positions' route
      // weights, which the down launch reads by position
      if (route_inl) {
        ri.rw_sorted = (float*)(ws + p.rws);
        r2.row_w = ri.rw_sorted;
        r2.row_w_by_idx = 0;
      }
    }
    const DecFuse f_up{fcnt, (long)p.N * (I / 128)};
    STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
          first_rc(
              [&] {
                return launch_stream_dec(2, 0, r1, sh_in ? &s1 : nullptr, k,
                                         L, p.up_items, st, p.bm,
                                         fused ? &f_up : nullptr,
                                         route_inl || perm_inl ? &ri : nullptr,
                                         nullptr, SF_FP8_F32S, p.sk_up);
              },
              [&] {
                return !fused && (p.ks_up > 1 || (sh_in && p.ks_up_sh > 1))
                           ? launch_split_finish(r1, sh_in ? &s1 : nullptr, L, st)
                           : 0;
              }));
    DecCombine dc{};
    if (comb_inl) {
      dc.cnt = fcnt + nfcnt; dc.inv = inv; dc.sorted = sorted;
      dc.y = y; dc.kstride = (long)p.N * H; dc.ks = p.ks_dn;
      dc.y_sh = sh_in ? y_sh : nullptr; dc.kstride_sh = (long)T * H;
      dc.ks_sh = sh_in ? p.ks_dn_sh : 0;
      dc.T = T; dc.H = H; dc.topk = k; dc.out_f32 = a->out_f32;
      dc.out = a->out;
    }
    STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
          launch_stream_dec(2, 1, r2, sh_in ? &s2 : nullptr, k, 0.f,
                            p.dn_items, st, p.bm, nullptr, nullptr,
                            comb_inl ? &dc : nullptr, SF_FP8_F32S, p.sk_dn));
    if (!sh || sh_in) {
      STAGE(clk, SLLM_MOE_STAGE_SHARED_UP, 0);
      STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN, 0);
    } else {
      STAGE(clk, SLLM_MOE_STAGE_SHARED_UP,
            first_rc(
                [&] {
                  return launch_stream_dec(1, 0, s1, nullptr, k, L,
                                           p.up_sh_items, st, p.bm_sh);
                },
                [&] {
                  return p.ks_up_sh > 1
                             ? launch_split_finish(s1, nullptr, L, st)
                             : 0;
                }));
      STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN,
            launch_stream_dec(1, 1, s2, nullptr, k, 0.f, p.dn_sh_items, st,
                              p.bm_sh));
    }
    STAGE(clk, SLLM_MOE_STAGE_COMBINE,
          comb_inl ? 0
                   : launch_combine_split(y, inv, k, y_sh, T, H, a->out_f32,
                                          a->out, p.ks_dn, (long)p.N * H,
                                          p.ks_dn_sh, (long)T * H, st));
  } else if (p.decode) {
    float* h = (float*)(ws + p.hq);
    float* y = (float*)(ws + p.y);
    STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
          launch_gemv(1, 1, a->x, 1, 1, sorted, k, p.N, tiles, ntiles,
          p.max_tiles, offsets, (const uint8_t*)a->w1, a->w1_s,
          (const uint8_t*)a->w3, a->w3_s, I, H, nullptr, L, h, st));
    STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
          launch_gemv(1, 0, h, 0, 0, sorted, k, p.N, tiles, ntiles, p.max_tiles,
          offsets, (const uint8_t*)a->w2, a->w2_s, nullptr, nullptr,
          H, I, w, 0.f, y, st));
    float* y_sh = nullptr;
    if (sh) {
      float* h_sh = (float*)(ws + p.hq_sh);
      y_sh = (float*)(ws + p.y_sh);
      STAGE(clk, SLLM_MOE_STAGE_SHARED_UP,
            launch_gemv(0, 1, a->x, 1, 0, nullptr, k, T, nullptr, nullptr, 1,
            nullptr, (const uint8_t*)a->s1, a->s1_s,
            (const uint8_t*)a->s3, a->s3_s, Is, H, nullptr, L, h_sh,
            st));
      STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN,
            launch_gemv(0, 0, h_sh, 0, 0, nullptr, k, T, nullptr, nullptr, 1,
            nullptr, (const uint8_t*)a->s2, a->s2_s, nullptr,
            nullptr, H, Is, nullptr, 0.f, y_sh, st));
    }
    STAGE(clk, SLLM_MOE_STAGE_COMBINE,
          launch_combine(y, 1, inv, k, y_sh, T, H, a->out_f32, a->out, st));
  } else {
    uint8_t* xq = (uint8_t*)(ws + p.xq);
    float* sx = (float*)(ws + p.sx);
    uint8_t* hq = (uint8_t*)(ws + p.hq);
    float* hs = (float*)(ws + p.hs);
    uint16_t* y = (uint16_t*)(ws + p.y);
    STAGE(clk, SLLM_MOE_STAGE_ACT_QUANT,
          rq_fused ? 0
                   : launch_act_quant((const uint16_t*)a->x, T, H, 1, xq, sx,
                                      nullptr, nullptr, st));
    uint16_t* y_sh = nullptr;
    uint8_t* hq_sh = nullptr;
    float* hs_sh = nullptr;
    if (sh) {
      hq_sh = (uint8_t*)(ws + p.hq_sh);
      hs_sh = (float*)(ws + p.hs_sh);
      y_sh = (uint16_t*)(ws + p.y_sh);
    }
    if (a->w13_packed) {
      SLLM_REQUIRE(a->w13_s_packed && a->w2_packed && a->w2_s_packed &&
                       (!sh || (a->s13_packed && a->s2_packed)),
                   "sllm_moe_ds_forward: packed weights incomplete");
      const long sh_rt = (T + 127) / 128;
      SegDesc r1{};
      r1.wreuse = weights_reused(p.N, E, PREFILL_BM);
      r1.a = xq; r1.sa = sx; r1.sorted_idx = sorted; r1.gather = 1;
      r1.tile_info = tiles; r1.num_tiles = ntiles; r1.max_tiles = p.max_tiles;
      r1.wp = (const uint8_t*)a->w13_packed; r1.s0 = a->w13_s_packed;
      r1.N = I; r1.K = H; r1.row_w = w; r1.row_w_by_idx = 1;
      r1.hq = hq; r1.hs = hs;
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
            dense ? launch_dense(0, r1, k, L, 1, st, device_cus())
                  : launch_stream(2, 0, r1, nullptr, k, L, 1,
                                  (long)p.max_tiles * (I / 128), st));
      SegDesc r2{};
      r2.wreuse = weights_reused(p.N, E, PREFILL_BM);
      r2.a = hq; r2.sa = hs; r2.sorted_idx = sorted; r2.gather = 0;
      r2.tile_info = tiles; r2.num_tiles = ntiles; r2.max_tiles = p.max_tiles;
      r2.wp = (const uint8_t*)a->w2_packed; r2.s0 = a->w2_s_packed;
      r2.N = H; r2.K = I; r2.y = y;
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
            dense ? launch_dense(1, r2, k, 0.f, 1, st, device_cus())
                  : launch_stream(2, 1, r2, nullptr, k, 0.f, 1,
                                  (long)p.max_tiles * (H / 256), st));
      if (sh) {
        SegDesc s1{};
        s1.wreuse = weights_reused(T, 1, PREFILL_BM);
        s1.a = xq; s1.sa = sx; s1.total_rows = T;
        s1.wp = (const uint8_t*)a->s13_packed; s1.s0 = a->s1_s; s1.s1 = a->s3_s;
        s1.N = Is; s1.K = H; s1.hq = hq_sh; s1.hs = hs_sh;
        // the shared expert's gate/up on the compute-dense FP8 kernel
        // (power-of-two scales as e8m0 MFMA scales) when its rows fill more
        // than one tile
        const bool sdense = dense8_mode() >= 1 && T > PREFILL_BM;
        STAGE(clk, SLLM_MOE_STAGE_SHARED_UP,
              sdense && dense8_fits(0, s1)
                  ? launch_dense8(0, s1, 0, k, L, 1, st, device_cus())
                  : launch_stream(1, 0, s1, nullptr, k, L, 1, sh_rt * (Is / 128),
                                  st));
        SegDesc s2{};
        s2.wreuse = weights_reused(T, 1, PREFILL_BM);
        s2.a = hq_sh; s2.sa = hs_sh; s2.total_rows = T;
        s2.wp = (const uint8_t*)a->s2_packed; s2.s0 = a->s2_s;
        s2.N = H; s2.K = Is; s2.y = y_sh;
        STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN,
              dense8_mode() == 2 && T > PREFILL_BM && dense8_fits(1, s2)
                  ? launch_dense8(1, s2, 0, k, 0.f, 1, st, device_cus())
                  : launch_stream(1, 1, s2, nullptr, k, 0.f, 1, sh_rt * (H / 256),
                                  st));
      }
    } else {
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_UP,
            launch_gemm1_mx(1, xq, sx, sorted, k, p.N, tiles, ntiles,
                            p.max_tiles, offsets, (const uint8_t*)a->w1,
                            a->w1_s, (const uint8_t*)a->w3, a->w3_s, I, H, w,
                            L, hq, hs, st));
      STAGE(clk, SLLM_MOE_STAGE_EXPERT_DOWN,
            launch_gemm2_mx(1, hq, hs, sorted, k, p.N, tiles, ntiles,
                            p.max_tiles, offsets, (const uint8_t*)a->w2,
                            a->w2_s, I, H, y, st));
      if (sh) {
        STAGE(clk, SLLM_MOE_STAGE_SHARED_UP,
              launch_gemm1_mx(0, xq, sx, nullptr, k, T, nullptr, nullptr, 0,
                              nullptr, (const uint8_t*)a->s1, a->s1_s,
                              (const uint8_t*)a->s3, a->s3_s, Is, H, nullptr,
                              L, hq_sh, hs_sh, st));
        STAGE(clk, SLLM_MOE_STAGE_SHARED_DOWN,
              launch_gemm2_mx(0, hq_sh, hs_sh, nullptr, k, T, nullptr, nullptr,
                              0, nullptr, (const uint8_t*)a->s2, a->s2_s, Is,
                              H, y_sh, st));
      }
    }
    STAGE(clk, SLLM_MOE_STAGE_COMBINE,
          launch_combine(y, 0, inv, k, y_sh, T, H, a->out_f32, a->out, st));
  }
  if (clk.finish()) return -1;
  return copy_debug(logits, w, ids, counts, sorted, inv, T, E, p.N,
                    a->logits_out, a->w_out, a->ids_out, a->counts_out,
                    a->sorted_out, a->inv_pos_out, st);
}

}  // extern "C"
