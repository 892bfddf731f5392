// Internal launchers shared between the library's translation units.
#pragma once
#include "common.h"

namespace sllm {

// ks > 1 (T <= 64 only; router_ksplit): the router GEMM writes ks partial
// logit slices T * E floats apart, and the routing launches given the same
// ks add them in order (storing the sum into slice 0). Split, the small
// router's shared-expert gate is left as ks partial logits at gate_out + T
// (T floats apart); a softmax routing launch given that buffer as gate
// adds them in order and writes the sigmoid to gate[0, T).
int router_ksplit(int T, int H);
// Prefill (T > 64) may also zero zero_n ints at zero: the permutation's
// chunk histograms, which a softmax routing launch given them as
// chunk_hist then fills (integer atomics: the counts do not depend on
// order), so that launch_permute(..., hist_ready = true) skips its
// histogram pass.
int launch_router_gemm(const uint16_t* x, const uint16_t* w, float* logits,
                       int T, int E, int H, hipStream_t st, int ks = 1,
                       int* zero = nullptr, long zero_n = 0);
// Per-token activation quantization run by the softmax routing launch
// (act_quant.h; x == nullptr: none).
struct ActQuant {
  const uint16_t* x;
  int H, pow2;
  uint8_t* q;
  float* s;
  const uint16_t* gate_w;
  float* gate_out;
};
// bias (E floats, or null): routing takes softmax top-k of logit + bias
// (the Qwen layer's per-expert routing bias); the logits stay as given.
int launch_route_softmax(const float* logits, float* w, int* ids, int T,
                         int E, int topk, float eps, hipStream_t st,
                         int ks = 1, float* gate = nullptr,
                         int* chunk_hist = nullptr,
                         const ActQuant* aq = nullptr,
                         const float* bias = nullptr);
// Fused prefill router (softmax routing, router_topk_fits): per token t
// and 128-expert tile y of the ny = ceil(E / 128) tiles, the tile's largest
// logit m and sum of exp(l - m) at stat[2 (t ny + y)] (+1), and its topk
// largest top-k keys, descending, at keys[(t ny + y) topk + j] (0 = none).
// launch_router_topk writes them (logits: null, or also the logits for the
// caller's copy) and zeroes zero_n ints at zero as launch_router_gemm.
// With q it also quantizes the activations into q / s (the activation-quant
// launch's layout and values), and with gate_w writes the shared-expert
// gate sigmoid(x . gate_w) to gate_out. launch_route_merge routes from the
// partials (filling chunk_hist as launch_route_softmax).
// router_part_bytes / router_part_at: the arrays' size and places in one
// buffer.
struct RouterPart {
  float* stat;
  uint64_t* keys;
  int topk;
  uint8_t* q;
  float* s;
  const uint16_t* gate_w;
  float* gate_out;
  int pow2;  // quantization scales rounded up to powers of two
  // keys mode: per-expert routing bias (E floats, or null) added to the
  // logits before the tiles' top-k and softmax partials (logits stays
  // without it)
  const float* bias;
};
bool router_topk_fits(int T, int E, int topk, int H);
size_t router_part_bytes(int T, int E, int topk);
RouterPart router_part_at(char* base, int T, int E, int topk);
int launch_router_topk(const uint16_t* x, const uint16_t* w, float* logits,
                       int T, int E, int H, const RouterPart& rp,
                       hipStream_t st, int* zero = nullptr, long zero_n = 0);
// The same launch in logits mode (DeepSeek prefill): the router logits,
// as launch_router_gemm writes them, and the activation quantization of
// launch_act_quant(x, T, H, pow2, q, s) in the same pass over x.
bool router_logits_quant_fits(int T, int H);
int launch_router_logits_quant(const uint16_t* x, const uint16_t* w,
                               float* logits, int T, int E, int H, uint8_t* q,
                               float* s, int pow2, hipStream_t st);
int launch_route_merge(const RouterPart& rp, int T, int E, float eps,
                       float* w, int* ids, hipStream_t st,
                       int* chunk_hist = nullptr);
// Decode-size helpers (router.hip): router GEMM for T <= 64 with an optional
// shared-expert gate tile, and softmax top-k fused with the permutation in
// one workgroup (when route_permute_small_fits).
// zero / nzero: ints cleared by the launch (the counters of a later
// launch on the stream), or none.
int launch_router_small_gate(const uint16_t* x, const uint16_t* w,
                             float* logits, int T, int E, int H,
                             const uint16_t* sgl, float* gate_out,
                             hipStream_t st, int ks = 1, int* zero = nullptr,
                             long nzero = 0);
bool route_permute_small_fits(int T, int E, int topk);
// zero / nzero (both permutation launches, one-workgroup path only): ints
// to clear on the way, the counters of the fused decode launches after it.
int launch_route_permute_small(const float* logits, float* w, int* ids, int T,
                               int E, int topk, float eps, int bm,
                               int* counts, int* offsets, int* sorted_idx,
                               int* inv_pos, int* tile_info, int* num_tiles,
                               int max_tiles, hipStream_t st, int ks = 1,
                               float* gate = nullptr, int* zero = nullptr,
                               int nzero = 0, const float* bias = nullptr);
int launch_route_grouped(const float* logits, const float* bias, float* w,
                         int* ids, int T, int E, int topk, int n_group,
                         int topk_group, int scoring, float route_scale,
                         hipStream_t st, int ks = 1);
int launch_route_hash(const float* logits, const int* token_ids,
                      const int* tid2eid, int vocab, float* w, int* ids,
                      int T, int E, int topk, int scoring, float route_scale,
                      hipStream_t st, int ks = 1);
// Multi-workgroup permutation: histograms of PERM_CHUNK assignments per
// chunk (chunk c, expert e at scratch int c E + e), used when
// permute_uses_chunk_hist(N, E) (otherwise one workgroup permutes).
constexpr int PERM_CHUNK = 1024;
bool permute_uses_chunk_hist(int N, int E);
size_t permute_scratch_bytes(int N, int E);
int launch_permute(const int* ids, int N, int E, int bm, int* counts,
                   int* offsets, int* sorted_idx, int* inv_pos,
                   int* tile_info, int* num_tiles, int max_tiles,
                   void* scratch, hipStream_t st, bool hist_ready = false,
                   int* zero = nullptr, int nzero = 0);
int launch_act_quant(const uint16_t* x, int T, int H, int pow2, uint8_t* q,
                     float* s, const uint16_t* gate_w, float* gate_out,
                     hipStream_t st);
int launch_gemm1_fp8(const uint8_t* xq, const float* sx, const int* sorted_idx,
                     int topk, int total_rows, const int* tile_info,
                     const int* num_tiles, int max_tiles, const int* offsets,
                     const uint8_t* wg, const float* wg_s, const uint8_t* wu,
                     const float* wu_s, int I, int H, const float* route_w,
                     float limit, int pow2, uint8_t* hq, float* hs,
                     hipStream_t st);
int launch_gemm2_fp8(const uint8_t* hq, const float* hs, const int* sorted_idx,
                     int topk, int total_rows, const int* tile_info,
                     const int* num_tiles, int max_tiles, const int* offsets,
                     const uint8_t* wd, const float* wd_s, int I, int H,
                     const float* row_w, uint16_t* y, hipStream_t st);
// MX-scaled grouped GEMMs (A e4m3 with power-of-two per-128 scales; B
// MXFP4 with e8m0 per 32, or FP8 with power-of-two 128x128 block scales).
int launch_gemm1_mx(int b_fp4, const uint8_t* xq, const float* sx,
                    const int* sorted_idx, int topk, int total_rows,
                    const int* tile_info, const int* num_tiles, int max_tiles,
                    const int* offsets, const uint8_t* w1, const void* w1_s,
                    const uint8_t* w3, const void* w3_s, int I, int H,
                    const float* route_w, float limit, uint8_t* hq, float* hs,
                    hipStream_t st);
int launch_gemm2_mx(int b_fp4, const uint8_t* hq, const float* hs,
                    const int* sorted_idx, int topk, int total_rows,
                    const int* tile_info, const int* num_tiles, int max_tiles,
                    const int* offsets, const uint8_t* w2, const void* w2_s,
                    int I, int H, uint16_t* y, hipStream_t st);
// Persistent weight-streaming grouped GEMM over packed weights
// (gemm_stream.hip). bf: 0 fp8 + fp32 scales, 1 fp8 + power-of-two scales,
// 2 MXFP4; mode 0: gate/up + SwiGLU + e4m3 re-quant, 1: down -> bf16 rows.
// Maximum of the ragged tile count sum_e ceil(n_e / bm) over N
// assignments to at most E experts: with t >= 1 touched experts,
// sum_e ceil(n_e / bm) = t + sum_e floor((n_e - 1) / bm) <= t + floor((N - t) / bm),
// which grows with t, so the maximum is m + floor((N - m) / bm) at
// m = min(E, N); m - 1 experts with one row and one with the rest reach it.
inline long tile_bound(long N, long E, int bm) {
  const long m = E < N ? E : N;
  return N <= 0 ? 0 : m + (N - m) / bm;
}
// Persistent grid of a streamed launch with at most upper_items items:
// #CUs rounded up to a multiple of 8 (one XCD slot each), grown until no
// workgroup is dealt more than max_items (an XCD's range holds at most
// ceil(upper / 8) items, dealt round-robin over its workgroups).
inline long stream_grid(long upper_items, int num_cus, int max_items) {
  const long per_xcd = (upper_items + 7) / 8;
  long nx = (num_cus + 7) / 8;
  const long need = (per_xcd + max_items - 1) / max_items;
  if (need > nx) nx = need;
  return 8 * nx;
}
// Most items one XCD receives when `total` items are dealt to the XCDs in
// chunks of `chunk` consecutive items (chunk c to XCD c % 8, the trailing
// partial chunk to XCD (total / chunk) % 8), as the decode kernel deals
// them: with ncf = total / chunk = 8a + r full chunks and a remainder
// crem, XCDs below r hold a + 1 chunks and XCD r holds a chunks + crem, so
// no XCD holds more than ceil(ceil(total / chunk) / 8) * chunk items. The
// bound does not decrease as total grows, so its value at an item bound
// covers every total up to that bound.
inline long chunked_xcd_share(long total, long chunk) {
  if (chunk < 1) chunk = 1;
  return ((total + chunk - 1) / chunk + 7) / 8 * chunk;
}
// Persistent grid of a chunk-dealt launch (moe_stream_dec_kernel) with at
// most upper_items items: #CUs rounded up to a multiple of 8, grown until
// an XCD's largest share, dealt round-robin over its workgroups, gives no
// workgroup more than max_items.
inline long stream_dec_grid(long upper_items, int num_cus, long chunk,
                            int max_items) {
  const long per_xcd = chunked_xcd_share(upper_items, chunk);
  long nx = (num_cus + 7) / 8;
  const long need = (per_xcd + max_items - 1) / max_items;
  if (need > nx) nx = need;
  return 8 * nx;
}

struct SegDesc {  // one segment (routed or shared expert) of a streamed launch
  const uint8_t* a;        // A rows (row stride K bytes)
  const float* sa;         // A scales (row stride K / 128)
  const int* sorted_idx;   // flat assignment index of permuted row p
  int gather;              // 1: A row of permuted row p is sorted_idx[p] / topk
  const int* tile_info;    // int4 per tile: expert, first row, rows, 0;
                           // null: identity rows [0, total_rows)
  const int* num_tiles;
  int max_tiles;           // host bound of *num_tiles (tile_info segments)
  int total_rows;
  const uint8_t* wp;       // packed weights
  const void* s0;          // fp8: fp32 scales of W1 / W2 (reference layout);
                           // fp4: packed e8m0 scales
  const void* s1;          // fp8 gate/up: fp32 scales of W3
  int N, K;
  const float* row_w;      // optional per-row weight (see row_w_by_idx)
  int row_w_by_idx;        // 1: row_w[sorted_idx[p]], 0: row_w[p]
  uint8_t* hq;             // mode 0 outputs at permuted row p
  float* hs;
  uint16_t* y;             // mode 1 output at permuted row p
  // decode split-K: each (row tile, column slab) item is cut into ksplit K
  // chunks (0 / 1: none) whose results land in slices pstride elements
  // apart -- mode 1 in y (summed by launch_combine_split), mode 0 in pp
  // (gate slices, then up slices; launch_split_finish writes h = SwiGLU of
  // the sums to hq for rows [0, total_rows))
  int ksplit;
  long pstride;
  float* pp;
  // prefill: 1 when the launch's experts average more rows than one row
  // tile, so that the weights are loaded through L2 (shared by an expert's
  // tiles) rather than streamed past it; the first segment decides for the
  // launch. Decode launches always stream.
  int wreuse;
};
// Items per XCD chunk of a decode launch of at most upper_items items, from
// its first segment: one row tile's items (column slabs of ntw columns x K
// chunks) for routed rows, so that the items of a tile, which read the same
// A rows, meet in one L2; an eighth of that for identity rows (the DeepSeek
// shared expert's launches, one row tile up to 16 or 32 tokens, whose A
// rows are a few KB per token), so that a one-tile launch still reaches all
// 8 XCDs (one-tile chunks left 7 of them idle: C4 B=1 shared gate/up 36.1
// us, down 27.2 us). Either way at most a 64th of the items, so that every
// XCD takes about 8 chunks: with few tiles of many items (a K-split launch
// at one token) whole-tile chunks gave one XCD twice the others' share (C4
// B=1 gate/up with the shared expert as a 9th tile: 56 K steps per
// workgroup against 32). The host passes it to the kernel and sizes the
// grid with it.
inline int dec_deal_chunk(int N, int ntw, int ksplit, bool routed,
                          long upper_items) {
  const int tile = (N / ntw) * (ksplit > 1 ? ksplit : 1);
  long c = routed ? tile : (tile + 7) / 8;
  c = std::min(c, upper_items / 64);
  return c > 1 ? (int)c : 1;
}
inline int dec_deal_chunk(const SegDesc& s, int ntw, long upper_items) {
  return dec_deal_chunk(s.N, ntw, s.ksplit, s.tile_info != nullptr,
                        upper_items);
}
// Stream-K deal of a decode launch (sk): its units (a row tile's column
// slab of a segment, routed units first) lie end to end on a line of cost
// (a unit costs its K steps times its weight w: 1, and 2 for the fp8
// segment of a mixed-format launch, whose steps stream twice the bytes);
// G equal ranges of that line go one to a workgroup, which takes the K
// steps whose start lies in its range (a unit's steps across two ranges are
// two items). An item's partial sums go to K slice (its range) - (the
// range of its unit's first step), of ks slices per unit; the unit's
// first item also writes zeros to the slices no range reached and counts
// them as arrivals, so that every unit holds ks slices, as a K-split unit
// does. Ranges are at least sk_lreq long, which keeps a unit within ks of
// them (and no range without a step of a unit it spans).
// (I: the kernel's deal takes them in 32-bit unsigned arithmetic, whose
// division is a short sequence where a 64-bit one runs to hundreds of
// scalar instructions: ten of them took 3.5 us of each launch)
template <class I = long>
__host__ __device__ inline I sk_lreq(int KB, int w, int ks) {
  const I l = ((I)(KB - 1) * (I)w + (I)(ks - 2)) / (I)(ks - 1);
  return l > (I)w ? l : (I)w;
}
// ranges over a line of cost C with grid workgroups
template <class I = long>
__host__ __device__ inline I sk_ranges(I C, I lreq, I grid) {
  const I g = C / lreq;
  return g < 1 ? 1 : (g < grid ? g : grid);
}
int launch_stream(int bf, int mode, const SegDesc& s0, const SegDesc* s1,
                  int topk, float limit, int pow2, long upper_items,
                  hipStream_t st);
// Compute-dense variant (gemm_dense.hip) for MXFP4 layers whose experts
// average more than one 128-row tile (wreuse): one routed segment with a
// tile table, N a multiple of 256 (gate/up) or 512 (down).
bool dense_fits(int bf, int mode, const SegDesc& s0, const SegDesc* s1);
// FP8 variant (gemm_dense8.hip): one segment, routed (tile table) or
// identity rows; f32s: fp32 block scales (else powers of two, applied as
// e8m0 MFMA scales); N a multiple of 128 (gate/up) or 256 (down), K <= 8192.
bool dense8_fits(int mode, const SegDesc& s0);
int launch_dense8(int mode, const SegDesc& s0, int f32s, int topk, float limit,
                  int pow2, hipStream_t st, int num_cus);
int launch_dense(int mode, const SegDesc& s0, int topk, float limit, int pow2,
                 hipStream_t st, int num_cus);
// Packed weight formats of the streamed launches (their bf argument): fp8
// with fp32 block scales, fp8 with power-of-two block scales, MXFP4.
enum { SF_FP8_F32S = 0, SF_FP8_POW2 = 1, SF_FP4 = 2 };
// Decode variant over the same packed weights: bm-row tiles (16 or 32; the
// tile_info rows must fit), weights converted to bf16 in registers and
// multiplied by unquantized activations with bf16 MFMAs. mode 0 reads bf16 rows (a, row stride K elements) and
// writes fp32 h rows to hq (as float*); mode 1 reads fp32 h rows (a as
// float*, split into bf16 hi + lo) and writes fp32 rows to y (as float*).
// bf: 0 / 1 fp8 (block scales applied in fp32), 2 MXFP4; bf1 (-1: bf): the
// second segment's format, which may differ only as MXFP4 first segment and
// fp8 second (a DeepSeek layer's routed and shared experts in one launch).
//
// A mode-0 decode launch may also finish its K-split items itself
// (DecFuse.cnt non-null): every workgroup, after its last item, counts its
// items' arrivals in cnt (zeroed earlier on the same stream) at
// cnt[row_begin (N / 128) + slab] (the second segment's from cnt1 on), and
// the workgroup whose arrival completes an item's K chunks computes its
// SwiGLU of the chunk sums as launch_split_finish does -- same arithmetic
// in the same order, so h equals that launch's bit for bit.
struct DecFuse {
  int* cnt;
  long cnt1;
};
// A mode-0 decode launch may also build its batch's permutation itself,
// from the ids of the routing launch (RouteInline.ids_in non-null), or
// route the batch too (RouteInline.logits non-null, Qwen softmax top-k, at
// most RI_MAX_ROUTE_T tokens: one per wave). Every workgroup computes the
// expert-major permutation (and before it the tokens' softmax top-k from
// the router's logits: ks K-chunk slices, plus bias) in LDS, before its
// items -- the arithmetic of the routing and permutation launches, so
// every workgroup holds the same tables, equal to theirs bit for bit.
// Workgroup 0 also writes them (w, ids when routing; counts, offsets,
// sorted, inv, tiles, ntiles) for the later launches, and finishes the
// split router's shared gate (gate non-null). The routed segment's
// tile_info / num_tiles / sorted_idx are then not read. Limits: E <=
// RI_MAX_E, T topk <= RI_MAX_N, max_tiles <= RI_MAX_TILES
// (route_inline_fits).
constexpr int RI_MAX_E = 512;
constexpr int RI_G = 4;                      // 64-assignment groups per wave
constexpr int RI_MAX_N = 8 * RI_G * 64;      // eight waves
constexpr int RI_MAX_TILES = 640;
constexpr int RI_MAX_ROUTE_T = 8;            // tokens routed in the launch
struct RouteInline {
  float* logits;
  const int* ids_in;
  const float* bias;
  float* gate;
  float* w;
  int* ids;
  int* counts;
  int* offsets;
  int* sorted;
  int* inv;
  int* tiles;
  int* ntiles;
  int T, E, topk, ks, nbits, bm, max_tiles;
  float eps;
  // grouped: the DeepSeek scored routing (route_grouped_token: scoring,
  // bias, n_group / topk_group limit, route_scale) in place of the Qwen
  // softmax top-k; E <= RI_MAX_E_GROUPED
  int grouped, scoring, n_group, topk_group;
  float route_scale;
  // optional, with logits (the batch routed in the launch): workgroup 0
  // also writes each sorted position's route weight (N floats), so that the
  // down launch reads its row weights by position
  float* rw_sorted;
};
constexpr int RI_MAX_E_GROUPED = 256;
bool route_inline_fits(int T, int E, int topk, long max_tiles);
// A mode-1 decode launch may also do the weighted combine (DecCombine.cnt
// non-null): its y slices go out as device-scope stores, every workgroup
// counts, after its last item, each of its item rows' arrival at
// cnt[t (H / 256) + slab] (zeroed earlier on the same stream), and the
// workgroup whose arrival completes a (token, 256-column slab) unit adds
// the unit's slices as launch_combine_split does -- the same partial sums
// in the same order, so out equals that launch's bit for bit.
struct DecCombine {
  int* cnt;
  const int* inv;     // inv_pos: permuted row of assignment t topk + j, or -1
  const int* sorted;  // sorted_idx: assignment of permuted row p
  const float* y;     // ks routed slices of N x H, kstride floats apart
  long kstride;
  int ks;
  const float* y_sh;  // ks_sh shared-expert slices of T x H, or null
  long kstride_sh;
  int ks_sh;
  int T, H, topk, out_f32;
  void* out;
};
inline long dec_combine_counters(long T, int H) { return T * (H / 256); }
int launch_stream_dec(int bf, int mode, const SegDesc& s0, const SegDesc* s1,
                      int topk, float limit, long upper_items,
                      hipStream_t st, int bm = 16,
                      const DecFuse* fuse = nullptr,
                      const RouteInline* route = nullptr,
                      const DecCombine* comb = nullptr, int bf1 = -1,
                      bool sk = false);
// Stream-K plan of a decode launch of nseg segments with units[i] units
// (row-tile bound x column slabs) of KB[i] K steps of weight w[i] (sk_lreq):
// K slices ks[i] (2..cap) that keep a unit within ks[i] ranges of the
// expected length; false when the deal cannot hold a workgroup's items.
bool dec_sk_plan(int nseg, const long* units, const int* KB, const int* w,
                 int cap, int* ks);
// The persistent grid of such a launch with ks[i] slices (0: the deal
// cannot hold a workgroup's items).
long dec_sk_launch_grid(int nseg, const long* units, const int* KB,
                        const int* w, const int* ks);
// Counter ints of a fused gate/up launch: N routed rows, T shared rows.
inline long dec_fuse_counters(long N, long T, int I, int Is) {
  return N * (I / 128) + T * (Is / 128);
}
// K chunks for a decode launch whose item count is at most upper_items
// over KB 128-wide K steps: down launches (dec_ksplit) and gate/up launches
// (dec_ksplit_up, which needs a finish launch and so splits only launches
// that would leave most CUs idle).
int dec_ksplit(long upper_items, int KB);
int dec_ksplit_up(long upper_items, int KB);
// Bound gate/up items below which the deal-based splits apply (larger
// decode batches stay unsplit: their split partials cost more than the
// balance gains).
constexpr long DEC_TARGET_ITEMS_DEALT = 768;
// Gate/up of a launch dealt in row-tile chunks (routed segment first, as the
// Qwen decode launch): the split of fewest steps for the busiest workgroup
// under the launch's own deal, for exp_items items (those a uniform routing
// touches) of a launch sized for upper_items, tile_items items per routed
// row tile unsplit; each split charged four steps (its finish). Batches of
// 768 bound items and more stay unsplit.
int dec_ksplit_up_dealt(long upper_items, long exp_items, long tile_items,
                        int KB);
// The down launch of the same deal: the split of fewest (steps + 1) per
// item over the busiest workgroup's items; no finish charge.
int dec_ksplit_dealt(long upper_items, long exp_items, long tile_items, int KB);
// Grid of a decode streamed launch of at most upper_items items dealt in
// chunks of `chunk` (dec_deal_chunk) on this device.
long dec_launch_grid(long upper_items, long chunk);
// h = silu(clamp(sum of gate slices)) * clamp(sum of up slices) for the
// split mode-0 segments (limit > 0: the SwiGLU clamp of the DeepSeek path).
int launch_split_finish(const SegDesc& s0, const SegDesc* s1, float limit,
                        hipStream_t st);
long packed_bytes(int fp4, int up, int E, int N, int K);
long packed_scale_bytes(int up, int E, int N, int K);

int launch_gemv(int wf, int swiglu, const void* act, int act_bf16,
                int gather_tokens, const int* sorted_idx, int topk,
                int total_rows, const int* tile_info, const int* num_tiles,
                int max_tiles, const int* offsets, const uint8_t* w0,
                const void* s0, const uint8_t* w1, const void* s1, int N,
                int K, const float* row_w, float limit, float* out,
                hipStream_t st);
int launch_combine(const void* y, int y_f32, const int* inv_pos, int topk,
                   const void* y_shared, int T, int H, int out_f32, void* out,
                   hipStream_t st);
// fp32 rows held as ks / ks_sh K-chunk slices kstride / kstride_sh
// elements apart (split-K decode); summed slice by slice in order. A null
// inv_pos is the identity permutation (slot j of token t at row t k + j).
int launch_combine_split(const float* y, const int* inv_pos, int topk,
                         const float* y_shared, int T, int H, int out_f32,
                         void* out, int ks, long kstride, int ks_sh,
                         long kstride_sh, hipStream_t st);

}  // namespace sllm
