/*
 * sllm_moe.h -- C-ABI of the MI355X (gfx950) mixture-of-experts library,
 * libsllm_moe.so. Plain pointers and sizes only.
 *
 * Conventions (as the reference's kernels/cuda/*.cu C-ABI):
 *   - every int-returning call returns 0 on success, -1 on bad arguments or
 *     a runtime error, -2 on a capacity bound; the message is available from
 *     the *_last_error getters (one thread-local buffer behind all of them);
 *   - "_dev" variants and all sllm_moe_* calls take DEVICE pointers, enqueue
 *     work and do not synchronise; the plain reference-named calls take HOST
 *     pointers and copy in and out;
 *   - `stream` arguments are hipStream_t (NULL = default stream);
 *   - bf16 tensors are passed as their uint16 bit patterns; e4m3 / e2m1 /
 *     e8m0 tensors as bytes.
 *
 * Reference file:line citations are relative to the skfine24/sLLM checkout.
 */
#ifndef SLLM_MOE_H
#define SLLM_MOE_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------- */
/* Errors                                                                 */
/* ---------------------------------------------------------------------- */
/* ref kernels/cuda/kernels.cu:27-29 (sllm_last_error) */
const char* sllm_last_error(void);
/* ref kernels/cuda/qwen4.cu:23-24 */
const char* sllm_q4_last_error(void);
/* ref kernels/cuda/fp8.cu:22-23 */
const char* sllm_fp8_last_error(void);
/* ref kernels/cuda/deepseek.cu:44 */
const char* sllm_ds_last_error(void);
/* new: same buffer, for the fused-layer entry points */
const char* sllm_moe_last_error(void);

/* ---------------------------------------------------------------------- */
/* Device buffers and sync (ref kernels/cuda/kernels.cu:31-194, 425)      */
/* ---------------------------------------------------------------------- */
/* ref kernels.cu:31 / kernels/_sllm_cuda.py:26 */
int sllm_device_count(void);
/* ref kernels.cu:150 / _sllm_cuda.py:48-49 */
void* sllm_buf_new(long nbytes);
/* ref kernels.cu:174 / _sllm_cuda.py:52-53 */
int sllm_buf_free(void* p);
/* ref kernels.cu:180 / _sllm_cuda.py:54-55 */
int sllm_buf_h2d(void* dst, const float* src, long nbytes);
/* ref kernels.cu:186 / _sllm_cuda.py:58-59 */
int sllm_buf_h2d_raw(void* dst, const void* src, long nbytes);
/* ref kernels.cu:191 / _sllm_cuda.py:56-57 */
int sllm_buf_d2h(float* dst, const void* src, long nbytes);
/* new: byte-typed D2H twin of sllm_buf_d2h for non-fp32 buffers */
int sllm_buf_d2h_raw(void* dst, const void* src, long nbytes);
/* ref kernels.cu:163 / _sllm_cuda.py:50-51 */
long sllm_mem_free_bytes(void);
/* ref kernels.cu:425 / _sllm_cuda.py:384-386 */
int sllm_sync(void);
/* new (no reference counterpart; the decode hook's host boundary, for
 * kernels/q4_device_decode.py:316-339 callers that pass host arrays):
 * page-locked host staging, stream-ordered copies in either direction
 * (hipMemcpyDefault), a stream wait, and fp32 -> bf16 bits on the host with
 * round to nearest even. */
void* sllm_host_new(long nbytes);
int sllm_host_free(void* p);
int sllm_copy_async(void* dst, const void* src, long nbytes, void* stream);
int sllm_stream_sync(void* stream);
int sllm_host_f32_to_bf16(void* dst, const float* src, long n);

/* ---------------------------------------------------------------------- */
/* Measurement and synthetic-data helpers (new; no reference counterpart:  */
/* the reference times with wall clocks only, bench/gpu_decode_timing.py)  */
/* ---------------------------------------------------------------------- */
/* hipEvent wrappers: time work on the stream the layer is launched on. */
void* sllm_event_new(void);
int sllm_event_free(void* ev);
int sllm_event_record(void* ev, void* stream);
int sllm_event_sync(void* ev);
/* milliseconds between two recorded events, -1 on error */
float sllm_event_elapsed_ms(void* start, void* stop);
/* stream-ordered byte fill (cache flushing between timed decode calls) */
int sllm_memset(void* dst, int value, long nbytes, void* stream);
/* stream-ordered device-to-device copy by a plain read/write kernel (the
 * reference copy of known size against which HBM byte counters are scaled);
 * dst, src 16-byte aligned */
int sllm_buf_copy(void* dst, const void* src, long nbytes, void* stream);
/* dst[i] ~ N(0, std^2), a pure function of (seed, i) */
int sllm_fill_normal(float* dst, long n, unsigned long long seed, float stdv,
                     void* stream);

/* ---------------------------------------------------------------------- */
/* Reference MoE kernel surface (ref kernels/cuda/qwen4.cu)                */
/* ---------------------------------------------------------------------- */
/* softmax -> top-k (ties to the lower id) -> renorm p/(sum p + 1e-20).
 * logits (n,E) f32 -> w (n,topk) f32, ids (n,topk) i32. E <= 2048,
 * topk <= 16. ref qwen4.cu:279-298 (host), :785-793 (_dev). */
int sllm_q4_moe_router(const float* logits, float* w_out, int* id_out, int n,
                       int E, int topk);
int sllm_q4_moe_router_dev(const float* logits, float* w_out, int* id_out,
                           int n, int E, int topk);
/* out = silu(g) * u, n floats. ref qwen4.cu:308-320, :795-799 */
int sllm_q4_swiglu(const float* g, const float* u, float* out, long n);
int sllm_q4_swiglu_dev(const float* g, const float* u, float* out, long n);
/* out (rows,O) f32 = A (rows,K) . W (O,K)^T, then post 1: silu(x/scale),
 * 2: sigmoid(x/scale). rows, K, O <= 0: -1. ref qwen4.cu:95-136 (host
 * pointers), :699-708 (_dev: device pointers). */
int sllm_q4_gemv_rows(const float* A, const float* W, float* out, int rows,
                      int K, int O, int post, float scale);
int sllm_q4_gemv_rows_dev(const float* A, const float* W, float* out, int rows,
                          int K, int O, int post, float scale);
/* out[t,:] += w[t] * y[t,:]. ref qwen4.cu:332-351, :801-806 */
int sllm_q4_axpy_rows(float* out, const float* y, const float* w, int n,
                      int H);
int sllm_q4_axpy_rows_dev(float* out, const float* y, const float* w, int n,
                          int H);
/* out[t,:] += sigmoid(g[t]) * shared[t,:]. ref qwen4.cu:363-382, :808-814 */
int sllm_q4_shared_gate_accum(float* out, const float* shared, const float* g,
                              int n, int H);
int sllm_q4_shared_gate_accum_dev(float* out, const float* shared,
                                  const float* g, int n, int H);

/* ---------------------------------------------------------------------- */
/* Reference GEMM surface                                                 */
/* ---------------------------------------------------------------------- */
/* C (M,N) = A (M,K) f32 . dequant(B)^T, B (N,K) e4m3, scale_inv
 * (ceil(N/bh), ceil(K/bw)) f32 with W[n,k] = e4m3(B[n,k]) * s[n/bh, k/bw]
 * (loaders/fp8.py:98-135). ref kernels/cuda/fp8.cu:72-110,
 * kernels/_fp8_cuda.py:87-112. */
int sllm_fp8_gemm(const float* A, const unsigned char* B,
                  const float* scale_inv, float* C, int M, int N, int K,
                  int block_h, int block_w);
int sllm_fp8_gemm_dev(const float* A, const unsigned char* B,
                      const float* scale_inv, float* C, int M, int N, int K,
                      int block_h, int block_w);
/* O (M,N) = A (M,K) . B (N,K)^T, fp32, B already dequantized (host
 * pointers). ref kernels/cuda/deepseek.cu:57-73. `scale`, `opts` unused. */
int sllm_ds_fp4_gemm(float* o, const float* a, const float* b, int M, int N,
                     int K, float scale, float* opts);
/* new: the same product with the FP4 bytes on the device: packed (N,K/2)
 * E2M1 (low nibble = even k) and (N, K/block_w) E8M0 scales
 * (loaders/fp8.py:177-200); replaces the host dequant of
 * kernels/_deepseek_cuda.py:89-94. Host / device pointer variants. */
int sllm_ds_fp4_gemm_packed(float* o, const float* a, const void* packed,
                            const void* scale_e8m0, int M, int N, int K,
                            int block_w);
int sllm_ds_fp4_gemm_packed_dev(float* o, const float* a, const void* packed,
                                const void* scale_e8m0, int M, int N, int K,
                                int block_w);
/* c (m,n) f32 = a (m,k) . w (n,k)^T, a and w both f32 (atype 0) or bf16
 * (atype 1); device pointers; c is fp32. ref kernels.cu:752-767
 * (cublasGemmEx), kernels/_sllm_cuda.py:503-506. */
int sllm_gemm_ex(const void* a, int atype, const void* w, void* c, int m,
                 int n, int k);
/* out = silu(g) * u for n fp32 elements of g and u (device pointers),
 * stored as fp32 (out_type 0) or bf16 (out_type 1). ref kernels.cu:897-919,
 * kernels/_sllm_cuda.py:529-532. */
int sllm_silu_mul(const void* g, const void* u, void* out, long n,
                  int out_type);

/* ---------------------------------------------------------------------- */
/* MoE building blocks (device pointers, stream-ordered, no sync)          */
/* ---------------------------------------------------------------------- */
/* logits (T,E) f32 = x (T,H) bf16 . W (E,H)^T bf16; H % 128 == 0.
 * replaces x @ router_w.T of ref/qwen4_exp.py:173 and the gemv of
 * kernels/q4_device_decode.py:322. */
int sllm_moe_router_gemm(const void* x_bf16, const void* w_bf16,
                         float* logits, int T, int E, int H, void* stream);
/* softmax top-k (ref/qwen4_exp.py:125-140); E <= 2048, topk <= 64. */
int sllm_moe_route_softmax(const float* logits, float* w_out, int* id_out,
                           int T, int E, int topk, float eps, void* stream);
/* scored routing with selection-only bias, optional group limit and
 * routed scaling (ref/deepseek_v4.py:522-561). scoring: 0 softmax,
 * 1 sigmoid, 2 sqrtsoftplus. n_group <= 1 disables the group limit. */
int sllm_moe_route_grouped(const float* logits, const float* bias,
                           float* w_out, int* id_out, int T, int E, int topk,
                           int n_group, int topk_group, int scoring,
                           float route_scale, void* stream);
/* hash-layer routing (ref/deepseek_v4.py:545-552, upstream
 * ref/hf_sources/dsv4/model.py:620-627): ids = tid2eid[clip(token_ids[t],
 * 0, vocab-1)] (tid2eid (vocab, topk) int32, table order, no bias), weights
 * = those experts' scores, renormalized unless softmax, times route_scale.
 * scoring as in sllm_moe_route_grouped; E <= 2048, topk <= 64.
 * Contract: every tid2eid entry lies in [0, E) (the reference raises
 * IndexError for larger ids). The kernel does not read out of bounds for a
 * bad entry: it writes the id through with a NaN weight (so the token's
 * renormalized weights are NaN), the permutation drops that assignment
 * (inv_pos -1) and the combine skips it. sllm_amd.moe.DeepseekMoE rejects
 * such tables on the host. */
int sllm_moe_route_hash(const float* logits, const int* token_ids,
                        const int* tid2eid, int vocab, float* w_out,
                        int* id_out, int T, int E, int topk, int scoring,
                        float route_scale, void* stream);
/* Stable expert-major permutation of ids (N = T*k int32) with a ragged tile
 * table of ceil(count/bm) row tiles per expert: tile_info holds max_tiles
 * int4 {expert, first permuted row, rows, 0}. new (the reference has no
 * permute; replaces the np.where grouping of ref/deepseek_v4.py:1080-1086).
 * scratch >= sllm_moe_permute_scratch_bytes(N, E). */
long sllm_moe_permute_scratch_bytes(int N, int E);
int sllm_moe_permute(const int* ids, int N, int E, int bm, int* counts,
                     int* offsets, int* sorted_idx, int* inv_pos,
                     int* tile_info, int* num_tiles, int max_tiles,
                     void* scratch, void* stream);
/* Per-1x128 e4m3 activation quant (ref/hf_sources/dsv4/kernel.py:40-125);
 * pow2 = 1 selects the ue8m0 power-of-two scale. Optional fused shared-
 * expert gate: gate_out[t] = sigmoid(x[t] . gate_w) (ref/qwen4_exp.py:182). */
int sllm_moe_act_quant(const void* x_bf16, int T, int H, int pow2,
                       void* q_e4m3, float* scale, const void* gate_w_bf16,
                       float* gate_out, void* stream);
/* out[t] = sum_j y[inv_pos[t*k+j]] + y_shared[t] (y rows bf16 or f32). */
int sllm_moe_combine(const void* y, int y_f32, const int* inv_pos, int topk,
                     const void* y_shared, int T, int H, int out_f32,
                     void* out, void* stream);
/* Streaming weight layout (gemm_stream.hip): a one-time repack of expert
 * weights into MFMA operand order so the prefill GEMMs read contiguous HBM.
 * fp4 = 0: w0 [, w1] are (E, N, K) e4m3; fp4 = 1: (E, N, K/2) packed e2m1
 * with (E, N, K/32) e8m0 scales s0 [, s1], whose packed copy goes to
 * out_scales. up = 1 packs a gate/up pair (N = intermediate, K = hidden,
 * N % 128 == 0), up = 0 a down weight (N = hidden, K = intermediate,
 * N % 256 == 0); K % 128 == 0. new: no reference counterpart. */
long sllm_moe_packed_bytes(int fp4, int up, int E, int N, int K);
long sllm_moe_packed_scale_bytes(int up, int E, int N, int K);
int sllm_moe_pack_weights(int fp4, int up, const void* w0, const void* w1,
                          const void* s0, const void* s1, int E, int N, int K,
                          void* out, void* out_scales, void* stream);
/* Streamed-GEMM health (new: no reference counterpart; the reference's
 * kernels have no work-item bound). The layer sizes each streamed launch's
 * persistent grid from a host bound of its work items, and a launch whose
 * bound is too small is refused (rc -2) before it runs. A workgroup that
 * still receives more items than it holds marks a per-device word and
 * leaves them undone; sllm_moe_stream_status synchronizes `stream`, returns
 * -2 (and clears the mark) if any launch did so since the last call, else 0.
 * sllm_moe_tile_bound is the bound of sum_e ceil(n_e / bm) for N
 * assignments over E experts; sllm_moe_stream_grid is the grid for an item
 * bound on num_cus CUs when each XCD takes a contiguous eighth of the
 * items, sllm_moe_stream_dec_grid when they are dealt to the XCDs in chunks
 * of `chunk` consecutive items (the decode kernel's deal); host-only
 * queries. */
int sllm_moe_stream_status(void* stream);
long sllm_moe_tile_bound(long N, int E, int bm);
long sllm_moe_stream_grid(long upper_items, int num_cus);
long sllm_moe_stream_dec_grid(long upper_items, int num_cus, long chunk);
/* Host plan query (new: no reference counterpart; no device work): what the
 * fused layer (deepseek = 0: sllm_moe_qwen_forward with packed FP8 weights,
 * 1: sllm_moe_ds_forward) plans for a shape. Is = 0: no shared expert.
 * out[0..9]: decode, bm (routed rows per tile), bm_sh, max_tiles, ks_r
 * (router K slices), ks_up, ks_up_sh, ks_dn, ks_dn_sh (decode K chunks),
 * #CUs used for planning; then, decode only, for the streamed launches
 * j = 0 gate/up, 1 down (Qwen: routed + shared segment), 2 and 3 the
 * DeepSeek shared expert's gate/up and down: out[10 + 3j] the launch's
 * item bound, out[11 + 3j] its XCD deal chunk (0: a stream-K deal, each
 * workgroup an equal range of the units' K steps), out[12 + 3j] its grid
 * (0 where a launch does not run). n_out >= SLLM_MOE_PLAN_FIELDS. */
#define SLLM_MOE_PLAN_FIELDS 22
int sllm_moe_plan_query(int deepseek, int T, int H, int E, int I, int Is,
                        int topk, int mode, int logits_given, long* out,
                        int n_out);
/* Synthetic-weight quantizers (data preparation): FP8 128x128 block
 * (s = amax/448, optionally its power-of-two ceiling) and MXFP4 per 32. */
int sllm_quantize_weight_fp8(const float* w, int N, int K, int pow2,
                             void* q_e4m3, float* scale, void* stream);
int sllm_quantize_weight_mxfp4(const float* w, int N, int K, void* packed,
                               void* scale_e8m0, void* stream);

/* ---------------------------------------------------------------------- */
/* Fused MoE layers                                                       */
/* ---------------------------------------------------------------------- */
/* mode: which arithmetic the expert products use */
#define SLLM_MOE_MODE_AUTO 0    /* decode when T <= 64, else prefill */
#define SLLM_MOE_MODE_PREFILL 1 /* e4m3 activations, grouped MFMA GEMMs */
#define SLLM_MOE_MODE_DECODE 2  /* fp32 activations, dequant GEMV */

/* Optional per-stage timing: when `stage_events` is non-NULL it points to
 * 2 * SLLM_MOE_STAGES hipEvent_t handles (from sllm_event_new); event 2s is
 * recorded on the layer's stream before stage s and 2s+1 after it. Stages
 * that do not run for a call record nothing. */
#define SLLM_MOE_STAGES 9
#define SLLM_MOE_STAGE_ROUTER_GEMM 0
#define SLLM_MOE_STAGE_ROUTE 1
#define SLLM_MOE_STAGE_PERMUTE 2
#define SLLM_MOE_STAGE_ACT_QUANT 3 /* activation quant + shared gate */
#define SLLM_MOE_STAGE_EXPERT_UP 4 /* routed gate/up (+SwiGLU) */
#define SLLM_MOE_STAGE_EXPERT_DOWN 5
#define SLLM_MOE_STAGE_SHARED_UP 6
#define SLLM_MOE_STAGE_SHARED_DOWN 7
#define SLLM_MOE_STAGE_COMBINE 8

/* Qwen-style layer (ref/qwen4_exp.py:153-184): softmax top-k routing,
 * SwiGLU experts with FP8 e4m3 weights and fp32 128x128 block scales
 * (orientation (ceil(out/128), ceil(in/128)), loaders/fp8.py:98-135),
 * optional shared expert with a sigmoid scalar gate.
 *   x (T,H) bf16; router_w (E,H) bf16 [or logits (T,E) f32 when
 *   logits_given]; wg/wu (E,I,H) + (E,I/128,H/128); wd (E,H,I) +
 *   (E,H/128,I/128); shared sg/su (Is,H), sd (H,Is) + scales; sgl (H) bf16.
 *   out (T,H) bf16 or f32. Optional debug copies: logits_out (T,E),
 *   w_out (T,k) f32, ids_out (T,k) i32, counts_out (E) i32. Prefill
 *   (T > 64, topk <= 16, H <= 4096) routes without materialising the
 *   logits; logits_out then makes the router launch write them as well.
 * Replaces qwen4_exp.moe_block_forward (the numpy oracle that runs today)
 * and kernels/q4_device_decode.py:316-339 (_moe). */
typedef struct sllm_moe_qwen_args {
  int T, H, E, I, Is, topk;
  int mode;
  int out_f32;
  int logits_given;
  int wdtype; /* 0: FP8 e4m3 + fp32 block scales; 1: bf16 (scales unused,
                 always the fp32-activation GEMV path) */
  float renorm_eps;
  const void* x;
  const float* logits;
  const void* router_w;
  const void* wg;
  const float* wg_s;
  const void* wu;
  const float* wu_s;
  const void* wd;
  const float* wd_s;
  const void* sg;
  const float* sg_s;
  const void* su;
  const float* su_s;
  const void* sd;
  const float* sd_s;
  const void* sgl;
  void* out;
  float* logits_out;
  float* w_out;
  int* ids_out;
  int* counts_out;
  void* workspace;
  long workspace_bytes;
  void* stream;
  void** stage_events;
  /* Optional packed weights (sllm_moe_pack_weights, fp8): when wgu_packed is
   * set the prefill path streams them (wd_packed, and for a shared expert
   * sgu_packed / sd_packed, must then be set too); the fp32 scale tensors
   * above are still read. */
  const void* wgu_packed; /* pack(up=1, wg, wu, E, I, H) */
  const void* wd_packed;  /* pack(up=0, wd, E, H, I) */
  const void* sgu_packed; /* pack(up=1, sg, su, 1, Is, H) */
  const void* sd_packed;  /* pack(up=0, sd, 1, H, Is) */
  /* Optional debug copies of the permutation the layer ran (N = T*k
   * assignments, flat index t*k + j): sorted_out (N) i32 the assignment at
   * each expert-major position, inv_pos_out (N) i32 each assignment's
   * position. Like the other debug outputs, asking for them keeps a
   * one-expert top-1 call on the routed path (which writes them). */
  int* sorted_out;
  int* inv_pos_out;
  /* Optional per-expert routing bias (E fp32 on the device, or NULL; new: no
   * reference counterpart -- the skewed-load configuration adds it to the
   * router logits of ref/qwen4_exp.py:173 before moe_route): every token
   * routes on softmax top-k of logits + router_bias, so the bias moves both
   * the selection and the weights. logits_out holds the logits without it. */
  const float* router_bias;
} sllm_moe_qwen_args;

long sllm_moe_qwen_workspace_bytes(const sllm_moe_qwen_args* a);
int sllm_moe_qwen_forward(const sllm_moe_qwen_args* a);
/* One layer call captured as a HIP graph and replayed (new; replaces the
 * 3k+5 launches and host round trips per layer and token of
 * kernels/q4_device_decode.py:316-339 for decode loops): the graph holds
 * every pointer and size of *a (x, out, workspace, weights; stream
 * ignored), so each replay runs the layer on the current contents of those
 * buffers. For decode batches the layer's launches dominate its time.
 * graph_new returns NULL on error (message in sllm_moe_last_error); stage
 * events cannot be captured. Launch orders a replay on `stream`. */
void* sllm_moe_qwen_graph_new(const sllm_moe_qwen_args* a);
int sllm_moe_graph_launch(void* graph, void* stream);
int sllm_moe_graph_free(void* graph);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): sllm_moe_qwen_forward with the library's own per-device
 * scratch (a fixed device array of sllm_moe_qwen_forward_noalloc_max_bytes()
 * = 32 MiB, held by every device the library runs on until the process
 * ends) in place of a workspace; a->workspace must be NULL and
 * a->workspace_bytes 0. Calls no hipMalloc / hipFree. A call whose
 * workspace (sllm_moe_qwen_workspace_bytes) exceeds the scratch returns -2
 * before any launch. Calls that overlap on one device share the scratch and
 * race: order them on one stream (or synchronize) per device. */
long sllm_moe_qwen_forward_noalloc_max_bytes(void);
int sllm_moe_qwen_forward_noalloc(const sllm_moe_qwen_args* a);

/* DeepSeek-style layer (ref/deepseek_v4.py:522-570 with the upstream
 * combine of ref/hf_sources/dsv4/model.py:684-699): scored routing with a
 * selection-only bias, optional group limit, routed scaling; routed experts
 * MXFP4 (w1/w3 (E,I,H/2) + (E,I,H/32) e8m0, w2 (E,H,I/2) + (E,H,I/32));
 * optional un-gated shared expert in FP8 with fp32 power-of-two 128x128
 * block scales (s1/s3 (Is,H), s2 (H,Is)); swiglu_limit clamps as
 * ref/deepseek_v4.py:564-570 (0 disables). */
typedef struct sllm_moe_ds_args {
  int T, H, E, I, Is, topk;
  int mode;
  int out_f32;
  int logits_given;
  int n_group, topk_group, scoring;
  float route_scale, swiglu_limit;
  const void* x;
  const float* logits;
  const void* router_w;
  const float* bias;
  const void* w1;
  const void* w1_s;
  const void* w3;
  const void* w3_s;
  const void* w2;
  const void* w2_s;
  const void* s1;
  const float* s1_s;
  const void* s3;
  const float* s3_s;
  const void* s2;
  const float* s2_s;
  void* out;
  float* logits_out;
  float* w_out;
  int* ids_out;
  int* counts_out;
  void* workspace;
  long workspace_bytes;
  void* stream;
  void** stage_events;
  /* Optional packed weights (sllm_moe_pack_weights) for the prefill path:
   * routed fp4 w1/w3 and w2 with their packed e8m0 scales, shared fp8. */
  const void* w13_packed;
  const void* w13_s_packed;
  const void* w2_packed;
  const void* w2_s_packed;
  const void* s13_packed;
  const void* s2_packed;
  /* Optional hash routing (the first n_hash_layers of DeepSeek-V4,
   * ref/deepseek_v4.py:545-552): with tid2eid (vocab, topk) int32 and the
   * tokens' ids token_ids (T) int32, routing takes the table's experts
   * instead of the biased top-k (see sllm_moe_route_hash). */
  const int* token_ids;
  const int* tid2eid;
  int vocab;
  /* Optional debug copies of the permutation, as in sllm_moe_qwen_args. */
  int* sorted_out;
  int* inv_pos_out;
} sllm_moe_ds_args;

long sllm_moe_ds_workspace_bytes(const sllm_moe_ds_args* a);
int sllm_moe_ds_forward(const sllm_moe_ds_args* a);

#ifdef __cplusplus
}
#endif
#endif /* SLLM_MOE_H */
