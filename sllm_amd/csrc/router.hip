// MoE router: logits GEMM and per-token top-k selection.
//
// Replaces kernels/cuda/qwen4.cu:229-298 + 785-793 (moe_router_kernel,
// sllm_q4_moe_router(_dev)) and the numpy routing of ref/qwen4_exp.py:
// 118-140 and ref/deepseek_v4.py:522-561.
//
// Design (gfx950): one wave64 per token. Lane l holds experts l, l+64, ...
// so each logits row is read with coalesced loads; softmax max/sum and the
// k rounds of arg-max are wave shuffles, never a serial thread-0 loop.
//
// Selection contract (bit-exact with the oracle):
// - softmax routing selects by the fp32 LOGIT, ties to the lower expert id.
//   Softmax is monotone, so this is the order of the exact probabilities;
//   the oracle's fp32 probabilities can only disagree where two different
//   logits round to the same probability (a certified rounding tie).
// - sigmoid routing selects by the fp32 biased score s + bias, where
//   s = fp32(1 / (1 + exp(-x))) is evaluated in fp64 as the reference does
//   (ref/deepseek_v4.py:526-528), ties to the lower expert id.
#include <algorithm>

#include "act_quant.h"
#include "launch.h"
#include "lds_dma.h"
#include "permute_fused.h"
#include "route_token.h"

namespace sllm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// --------------------------------------------------------------------------
// router GEMM: logits (T, E) fp32 = x (T, H) bf16 . W (E, H)^T bf16
// --------------------------------------------------------------------------
// MFMA 16x16x32 bf16; lane l feeds row l % 16 and the 8 K values
// [8 (l / 16), +8) of each 32-wide K slice (the same lane->K assignment for
// both operands, so the MFMA's internal K order does not matter). Output:
// lane l, element v = row 4 (l / 16) + v, column l % 16.
//
// Prefill (T > 64): a workgroup owns a 64-token x 128-expert tile; both
// operands go through LDS in 128-wide K chunks (row stride padded to
// 272 B). Three register stages keep three chunks' global loads in flight
// (the loads are L2 hits for the most part, so the kernel is bound by their
// latency, not by bytes) while two LDS buffers alternate between store and
// multiply. Eight waves: wave (wm, we) of the 2 x 4 arrangement computes
// 32 tokens x 32 experts as 2 x 2 subtiles (eight waves rather than four:
// 18.5 against 20.7 us at 4096 x 512 x 2048). x is read E / 128 times and
// W T / 64 times, both mostly from L2. Waves of 32 x 64 over half of each
// chunk's K (a quarter fewer LDS fragment reads, the halves added through
// LDS at the end) measured no faster: 20.9 against 21.5 us.
constexpr int RG_TT = 64, RG_TE = 128, RG_KC = 128, RG_LS = 136;  // LS in bf16
constexpr int RG_NS = 3;  // register stages (prefetch distance in chunks)

__global__ __launch_bounds__(512, 1) void router_gemm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    float* __restrict__ logits, int T, int E, int H, int* __restrict__ zero,
    long zero_n) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][RG_TT * RG_LS];
  __shared__ __attribute__((aligned(16))) uint16_t ws[2][RG_TE * RG_LS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  {  // the permutation's chunk histograms, filled by the routing launch
    const long nthr = (long)gridDim.x * gridDim.y * 512;
    for (long i = ((long)blockIdx.y * gridDim.x + blockIdx.x) * 512 + tid;
         i < zero_n; i += nthr)
      zero[i] = 0;
  }
  const int lr = lane & 15, lg = lane >> 4;
  const int wm = wave >> 2, we = wave & 3;
  const int t0 = blockIdx.x * RG_TT, e0 = blockIdx.y * RG_TE;
  // global -> register staging, 16 threads per 256-byte row segment:
  // x 64 rows (2 x 16 B per thread), W 128 rows (4 x 16 B per thread)
  const int srow = tid >> 4, scol = (tid & 15) * 8;  // scol in bf16
  const uint16_t* xg = x + (size_t)min(t0 + srow, T - 1) * H + scol;
  const uint16_t* wg = w + (size_t)min(e0 + srow, E - 1) * H + scol;
  int xro[2], wro[4];
#pragma unroll
  for (int q = 0; q < 2; ++q)
    xro[q] = (min(t0 + srow + 32 * q, T - 1) - min(t0 + srow, T - 1)) * H;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    wro[q] = (min(e0 + srow + 32 * q, E - 1) - min(e0 + srow, E - 1)) * H;
  u32x4 r[RG_NS][6];
  auto gload = [&](u32x4 (&rg)[6], int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q) rg[q] = *(const u32x4*)(xg + xro[q] + k0);
#pragma unroll
    for (int q = 0; q < 4; ++q) rg[2 + q] = *(const u32x4*)(wg + wro[q] + k0);
  };
  auto sstore = [&](const u32x4 (&rg)[6], int b) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      *(u32x4*)(xs[b] + (srow + 32 * q) * RG_LS + scol) = rg[q];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *(u32x4*)(ws[b] + (srow + 32 * q) * RG_LS + scol) = rg[2 + q];
  };
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  auto mma = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8 a[2], bb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *(const bf16x8*)(xs[b] + (wm * 32 + i * 16 + lr) * RG_LS + q * 32 + lg * 8);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bb[j] = *(const bf16x8*)(ws[b] + (we * 32 + j * 16 + lr) * RG_LS + q * 32 + lg * 8);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bb[j], acc[i][j], 0, 0, 0);
    }
  };
  const int nk = H / RG_KC;
  // chunk kc lives in register stage kc % 3 and LDS buffer kc % 2. A step
  // stores its chunk, waits at the barrier (every wave is then done with the
  // other LDS buffer's multiply of the step before), refills its register
  // stage with chunk kc + 3 and multiplies. Main-loop prefetches past the
  // last chunk re-read it (unconditional loads keep the wait counts exact);
  // the tail steps load only what exists.
  auto kof = [&](int kc) { return min(kc, nk - 1) * RG_KC; };
  auto step = [&](u32x4 (&rg)[6], int b, int kc) __attribute__((always_inline)) {
    sstore(rg, b);
    __syncthreads();
    gload(rg, kof(kc + RG_NS));
    mma(b);
  };
  auto tail_step = [&](u32x4 (&rg)[6], int b, int kc) __attribute__((always_inline)) {
    sstore(rg, b);
    __syncthreads();
    if (kc + RG_NS < nk) gload(rg, kc * RG_KC + RG_NS * RG_KC);
    mma(b);
  };
#pragma unroll
  for (int s0 = 0; s0 < RG_NS; ++s0) gload(r[s0], kof(s0));
  int kc = 0;
  for (; kc + 6 <= nk; kc += 6) {
    step(r[0], 0, kc);
    step(r[1], 1, kc + 1);
    step(r[2], 0, kc + 2);
    step(r[0], 1, kc + 3);
    step(r[1], 0, kc + 4);
    step(r[2], 1, kc + 5);
  }
  if (kc < nk) tail_step(r[0], 0, kc);
  if (kc + 1 < nk) tail_step(r[1], 1, kc + 1);
  if (kc + 2 < nk) tail_step(r[2], 0, kc + 2);
  if (kc + 3 < nk) tail_step(r[0], 1, kc + 3);
  if (kc + 4 < nk) tail_step(r[1], 0, kc + 4);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int rr = t0 + wm * 32 + i * 16 + lg * 4 + v;
        const int c = e0 + we * 32 + j * 16 + lr;
        if (rr < T && c < E) logits[(size_t)rr * E + c] = acc[i][j][v];
      }
}

// Small T (decode, T <= 64): a workgroup owns 16 experts and all T tokens;
// its 8 waves split K (wave w takes the 32-wide slices w, w + 8, ...) so the
// router weights stream through many CUs at once; partial sums are reduced
// through LDS.
constexpr int RG_SMALL_T = 64;

// Decode-size router GEMM: workgroup (x, q) computes experts [16 x, +16)
// over K chunk q of gridDim.y (32-wide K slices split evenly), all NTI
// 16-token tiles, and writes its partial logits to slice q (q T E floats
// in); the routing kernels add the slices in order. With gate_out, an
// extra column of workgroups (x = E / 16) computes the shared-expert gate
// logit x . sgl of every token over the same K chunks (its 16 weight rows
// all read sgl; column 0 is kept): unsplit it writes sigmoid(logit) to
// gate_out[t], split it writes chunk q's partial to gate_out[T + q T + t]
// and the routing kernel adds the partials in order and applies the
// sigmoid (route_gate_finish). zero[0, nzero) is cleared (a later
// launch's counters).
template <int NTI>
__global__ __launch_bounds__(512) void router_gemm_small_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    float* __restrict__ logits, int T, int E, int H,
    const uint16_t* __restrict__ sgl, float* __restrict__ gate_out,
    int* __restrict__ zero, long nzero) {
  __shared__ float part[8][NTI * 16][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (long i = ((long)blockIdx.y * gridDim.x + blockIdx.x) * 512 + threadIdx.x;
       i < nzero; i += (long)gridDim.x * gridDim.y * 512)
    zero[i] = 0;
  const int lr = lane & 15, lg = lane >> 4;
  const int e0 = blockIdx.x * 16;
  const bool gate_tile = e0 >= E;
  const int nsl = H / 32, ks = gridDim.y, q = blockIdx.y;
  const int s0 = q * nsl / ks, s1 = (q + 1) * nsl / ks;
  const uint16_t* brow = (gate_tile ? sgl : w + (size_t)min(e0 + lr, E - 1) * H) + lg * 8;
  const uint16_t* arow[NTI];
#pragma unroll
  for (int i = 0; i < NTI; ++i)
    arow[i] = x + (size_t)min(i * 16 + lr, T - 1) * H + lg * 8;
  f32x4 acc[NTI];
#pragma unroll
  for (int i = 0; i < NTI; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // the wave's K slices (s0 + w, s0 + w + 8, ...) in groups of 4, all loads
  // of a group in flight together (rows past T re-read row T - 1; slices
  // past the chunk are clamped and skipped)
  for (int g0 = s0 + wave; g0 < s1; g0 += 32) {
    bf16x8 b[4], a[4][NTI];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k0 = min(g0 + 8 * j, s1 - 1) * 32;
      b[j] = *(const bf16x8*)(brow + k0);
#pragma unroll
      for (int i = 0; i < NTI; ++i) a[j][i] = *(const bf16x8*)(arow[i] + k0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (g0 + 8 * j < s1) {
#pragma unroll
        for (int i = 0; i < NTI; ++i)
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j][i], b[j], acc[i], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NTI; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wave][i * 16 + lg * 4 + v][lr] = acc[i][v];
  __syncthreads();
  float* out = logits + (size_t)q * T * E;
  for (int qq = threadIdx.x; qq < T * 16; qq += 512) {
    const int r = qq >> 4, c = qq & 15;
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < 8; ++wv) s += part[wv][r][c];
    if (gate_tile) {
      if (c == 0) {
        if (ks == 1) gate_out[r] = sigmoid_f32(s);
        else gate_out[T + q * T + r] = s;
      }
    } else if (e0 + c < E) {
      out[(size_t)r * E + e0 + c] = s;
    }
  }
}

// --------------------------------------------------------------------------
// fused prefill router (softmax routing): router GEMM, each 128-expert
// tile's top-k and softmax partials, activation quantization
// --------------------------------------------------------------------------
// Maximum / sum over each 16-lane row, in every lane of the row (the first
// four DPP steps of wave_max / wave_sum: all lanes add in the same order).
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v, 0u));
  v = max(v, dpp_u32<0x4E>(v, 0u));
  v = max(v, dpp_u32<0x141>(v, 0u));
  return max(v, dpp_u32<0x140>(v, 0u));
}

__device__ __forceinline__ float row16_max(float v) {
  const uint32_t ni = __float_as_uint(-INFINITY);
  v = fmaxf(v, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x141>(__float_as_uint(v), ni)));
  return fmaxf(v, __uint_as_float(dpp_u32<0x140>(__float_as_uint(v), ni)));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x141>(__float_as_uint(v), 0u));
  return v + __uint_as_float(dpp_u32<0x140>(__float_as_uint(v), 0u));
}

// Descending top-k (topk <= 16) of two tokens' keys per 16-lane row (key[h],
// 8 per lane, 0 = none, distinct): pick j of token h goes to kl[h][j]. The
// two tokens' picks interleave (independent reduction chains). Every pick
// is the maximum of the row's lane heads, found on the value halves; only
// when some row holds its maximum value on two lanes (a ballot shows it)
// are the low halves (the lower expert id) compared among them. The lane
// holding the pick stores and pops it.
__device__ __forceinline__ void row16_topk_keys2(uint64_t (&key)[2][8],
                                                 int topk, uint64_t* kl0,
                                                 uint64_t* kl1) {
  sort_desc<8>(key[0]);
  sort_desc<8>(key[1]);
  for (int kk = 0; kk < topk; ++kk) {
    uint32_t hi[2], mhi[2];
    bool own[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) hi[h] = (uint32_t)(key[h][0] >> 32);
#pragma unroll
    for (int h = 0; h < 2; ++h) mhi[h] = row16_max_u32(hi[h]);
#pragma unroll
    for (int h = 0; h < 2; ++h) own[h] = hi[h] == mhi[h];
    if (__popcll(__ballot(own[0])) != 4 || __popcll(__ballot(own[1])) != 4) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t mlo = row16_max_u32(own[h] ? (uint32_t)key[h][0] : 0u);
        own[h] = own[h] && (uint32_t)key[h][0] == mlo;
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (own[h]) {
        (h ? kl1 : kl0)[kk] = key[h][0];
#pragma unroll
        for (int i = 0; i < 7; ++i) key[h][i] = key[h][i + 1];
        key[h][7] = 0;
      }
    }
  }
}

constexpr int RT_XB = RG_TT * 256;                 // x chunk: 64 rows x 256 B
constexpr int RT_WB = RG_TE * 256;                 // W chunk: 128 rows x 256 B
constexpr int RT_STAGE = RT_XB + RT_WB;            // 48 KB, three stages
constexpr int RT_LOADS = RT_STAGE / (512 * 16);    // 6 loads / thread / stage
constexpr int RT_GATE_MAX = 4096;                  // gate weights in LDS
constexpr int RG_LT = 132;  // row stride (floats) of the tile's logits in LDS

// LDS byte offset of 16-byte chunk c (columns [8 c, +8)) of row r of a
// 256-byte-row tile: the chunk index is XOR-swizzled with the row's low
// four bits, so the 16 rows an MFMA fragment read takes (one chunk of
// each) fall on 16 different bank groups.
__device__ __forceinline__ int rt_off(int r, int c) {
  return r * 256 + ((c ^ (r & 15)) << 4);
}

// Fused prefill router (RouterPart): workgroup (bx, y) computes the logits
// of tokens [64 bx, +64) x experts [128 y, +128) as router_gemm_kernel's
// waves do (2 x 4 waves of 32 x 32, MFMA 16x16x32 bf16), with the operands
// brought into LDS by direct-to-LDS loads: three 48 KB stages, two K chunks
// in flight ahead of the one multiplied, every thread issuing six 16-byte
// loads per stage (slot p = 512 j + tid of the stage holds x row p / 16 for
// p < 1024, else W row (p - 1024) / 16, chunk (p % 16) ^ (row % 16)).
//
// Activation quantization (rp.q): chunk kc of the x tile is quantization
// block kc of each row (act_quant.h: the same operations, so the same
// codes and scales); tile column y quantizes rows [qr0, qr1) (its share,
// 64 / ny) of every chunk while the chunk is in LDS: x is not read again
// and every step gets the same share. A 16-lane row per x row, 8 columns
// per lane. rp.gate_w: the same lanes form those rows' shared-expert gate
// logits (gate weights copied to LDS once), each lane adding its columns'
// products chunk by chunk, then the row's lanes (row16_sum);
// gate_out[t] = sigmoid(logit).
//
// Logits mode (rp.keys null; DeepSeek's grouped routing): the logits go
// out as router_gemm_kernel writes them (the same MFMA order, so the same
// values) and the quantization is the launch's other output (rp.pow2:
// power-of-two scales).
//
// Epilogue: the tile's logits go to LDS (logits, when not null, also gets
// them for the caller's copy); each wave takes 8 tokens, two per 16-lane
// row (row lane r holds experts e0 + r + 16 i, i < 8): the tile's maximum
// m, sum of exp(l - m) and top-k keys (row16_topk_keys2). The sum takes
// the hardware exponential (__expf): it only normalises the probabilities,
// whose scale cancels in the weights p_j / (sum of the picks' p); the
// picks' own probabilities take expf.
__global__ __launch_bounds__(512, 1) void router_topk_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    float* __restrict__ logits, int T, int E, int H, int* __restrict__ zero,
    long zero_n, RouterPart rp) {
  __shared__ __attribute__((aligned(16))) uint8_t stg0[RT_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stg1[RT_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stg2[RT_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t gsl[RT_GATE_MAX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  {  // the permutation's chunk histograms, filled by the routing launch
    const long nthr = (long)gridDim.x * 512;
    for (long i = (long)blockIdx.x * 512 + tid; i < zero_n; i += nthr)
      zero[i] = 0;
  }
  // Tile (bx, by) of workgroup b (router_topk_grid): XCD b % 8 takes token
  // tiles b % 8, b % 8 + 8, ..., each one's ny expert tiles on consecutive
  // workgroups of that XCD, so a token tile's activation rows come from HBM
  // once and from the XCD's L2 for its other expert tiles. (With the token
  // tile as the fast grid dimension, the expert tiles of one token tile ran
  // a whole round of the grid apart once T passed 64 x #CUs / ny tokens,
  // each reading the rows again: 16384 tokens x 512 experts fetched 286 MB
  // for 67 MB of activations; with this deal 127 MB. The launch's time did
  // not change (105 us): it is bound by its MFMA and top-k work, not HBM.)
  const int ny = (E + RG_TE - 1) / RG_TE, ntx = (T + RG_TT - 1) / RG_TT;
  const int bx = (int)(blockIdx.x % 8) + 8 * (int)(blockIdx.x / 8 / ny);
  const int by = (int)(blockIdx.x / 8 % ny);
  if (bx >= ntx) return;  // the last XCD round's spare workgroups
  const int t0 = bx * RG_TT, e0 = by * RG_TE;
  const int nk = H / RG_KC;
  auto stage = [&](int kc) __attribute__((always_inline)) -> uint8_t* {
    const int sidx = kc % 3;
    return sidx == 0 ? stg0 : sidx == 1 ? stg1 : stg2;
  };
  const uint16_t* src[RT_LOADS];
#pragma unroll
  for (int j = 0; j < RT_LOADS; ++j) {
    const int p = 512 * j + tid;
    if (p < RT_XB / 16) {
      const int r = p >> 4, c = (p & 15) ^ (r & 15);
      src[j] = x + (size_t)min(t0 + r, T - 1) * H + c * 8;
    } else {
      const int q = p - RT_XB / 16, r = q >> 4, c = (q & 15) ^ (r & 15);
      src[j] = w + (size_t)min(e0 + r, E - 1) * H + c * 8;
    }
  }
  auto issue = [&](int kc) __attribute__((always_inline)) {
    uint8_t* base = stage(kc) + wave * 1024;
#pragma unroll
    for (int j = 0; j < RT_LOADS; ++j)
      dma::to_lds(src[j] + kc * RG_KC, base + j * 8192, 16);
  };
  issue(0);
  if (nk > 1) issue(1);
  const bool quant_on = rp.q != nullptr, gate_on = rp.gate_w != nullptr;
  if (gate_on) {  // visible to every wave after the first step's barrier
    for (int i = tid * 8; i < H; i += 512 * 8)
      *(u32x4*)(gsl + i) = *(const u32x4*)(rp.gate_w + i);
  }
  const int lr = lane & 15, lg = lane >> 4;
  const int wm = wave >> 2, we = wave & 3;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int rpy = (RG_TT + ny - 1) / ny;
  const int qr0 = min(RG_TT, by * rpy), qr1 = min(RG_TT, qr0 + rpy);
  const int qslot = tid >> 4, q16 = tid & 15;
  float gdot[2] = {0.f, 0.f};
  // a step's quantized rows are stored at the start of the next step,
  // before that step's loads: the loads then remain the newest memory
  // operations whenever a step waits, so each wait is for its own stage
  uint2 qpk[2];
  float qsc[2];
  int qkc = -1;
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int r = qr0 + qslot + 32 * ps;
      if (qkc >= 0 && r < qr1 && t0 + r < T) {
        const int t = t0 + r;
        *(uint2*)(rp.q + (size_t)t * H + qkc * RG_KC + q16 * 8) = qpk[ps];
        if (q16 == 0) rp.s[(size_t)t * (H / RG_KC) + qkc] = qsc[ps];
      }
    }
  };
  for (int kc = 0; kc < nk; ++kc) {
    // this thread's loads of chunk kc are done once at most the six of
    // chunk kc + 1 are outstanding; the barrier makes every thread's done
    if (kc + 1 < nk) dma::wait_vm<RT_LOADS>();
    else dma::wait_vm<0>();
    dma::bar_lds();
    if (quant_on) flush();
    // stage (kc + 2) % 3 was last read in step kc - 1, which every wave
    // finished before the barrier
    if (kc + 2 < nk) issue(kc + 2);
    const uint8_t* sx = stage(kc);
    const uint8_t* sw = sx + RT_XB;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8 a[2], bb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *(const bf16x8*)(sx + rt_off(wm * 32 + i * 16 + lr, q * 4 + lg));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bb[j] = *(const bf16x8*)(sw + rt_off(we * 32 + j * 16 + lr, q * 4 + lg));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bb[j], acc[i][j], 0, 0, 0);
    }
    if (quant_on) {
#pragma unroll
      for (int ps = 0; ps < 2; ++ps) {
        const int r = qr0 + qslot + 32 * ps;  // the same on the row's 16 lanes
        if (r >= qr1) continue;
        const u32x4 raw = *(const u32x4*)(sx + rt_off(r, q16));
        const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
        float v[8];
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = __uint_as_float(wd[i] << 16);
          v[2 * i + 1] = __uint_as_float(wd[i] & 0xFFFF0000u);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = row16_max(amax);
        if (gate_on) {
          const u32x4 gr = *(const u32x4*)(gsl + kc * RG_KC + q16 * 8);
          const uint32_t gd[4] = {gr.x, gr.y, gr.z, gr.w};
          float gsum = gdot[ps];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            gsum += v[2 * i] * __uint_as_float(gd[i] << 16);
            gsum += v[2 * i + 1] * __uint_as_float(gd[i] & 0xFFFF0000u);
          }
          gdot[ps] = gsum;
        }
        float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
        if (rp.pow2) sc = pow2_ceil(sc);
        // x / sc correctly rounded without a division per value (Markstein:
        // with ry = RN(1 / sc), q0 = RN(x ry) and the exact residual
        // r = x - q0 sc (one FMA), RN(q0 + r ry) = RN(x / sc) while no
        // value under- or overflows, and x's sign restores -0 / sc = -0);
        // the IEEE divisions' VCC-serialised sequences cost 2.5 us of this
        // launch at 4096 x 2048. tests/test_quant_division.py checks the
        // formula against IEEE division exhaustively over bf16 inputs.
        const float ry = 1.0f / sc;
        float yq[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float q0 = v[i] * ry;
          const float rr = __builtin_fmaf(-q0, sc, v[i]);
          const float qt = __builtin_copysignf(__builtin_fmaf(rr, ry, q0), v[i]);
          yq[i] = fminf(fmaxf(qt, -448.f), 448.f);
        }
        qpk[ps].x = f32x4_to_e4m3(yq[0], yq[1], yq[2], yq[3]);
        qpk[ps].y = f32x4_to_e4m3(yq[4], yq[5], yq[6], yq[7]);
        qsc[ps] = sc;
      }
      qkc = kc;
    }
  }
  if (quant_on) flush();
  if (gate_on) {
#pragma unroll 1
    for (int ps = 0; ps < 2; ++ps) {
      const int r = qr0 + qslot + 32 * ps;
      if (r >= qr1) break;
      const float g = row16_sum(gdot[ps]);
      if (q16 == 0 && t0 + r < T) rp.gate_out[t0 + r] = sigmoid_f32(g);
    }
  }
  if (!rp.keys) {  // logits mode: the logits for a routing launch of its own
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = wm * 32 + i * 16 + lg * 4 + v, c = we * 32 + j * 16 + lr;
          if (t0 + r < T && e0 + c < E)
            logits[(size_t)(t0 + r) * E + e0 + c] = acc[i][j][v];
        }
    return;
  }
  dma::bar_lds();  // every wave is done with the last chunk
  float* lt = reinterpret_cast<float*>(stg0);
  uint64_t* kl = reinterpret_cast<uint64_t*>(stg1);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = wm * 32 + i * 16 + lg * 4 + v, c = we * 32 + j * 16 + lr;
        // routing takes logit + bias (rp.bias: the per-expert routing
        // bias); the caller's copy gets the logit itself
        lt[r * RG_LT + c] = rp.bias && e0 + c < E ? acc[i][j][v] + rp.bias[e0 + c]
                                                  : acc[i][j][v];
        if (logits && t0 + r < T && e0 + c < E)
          logits[(size_t)(t0 + r) * E + e0 + c] = acc[i][j][v];
      }
  dma::bar_lds();
  const int r16 = lane & 15, rg = lane >> 4;
  const int y = by;
  int tl[2];
  float m[2], sm[2];
  uint64_t key[2][8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    tl[h] = wave * 8 + 4 * h + rg;
    float v[8];
    float mm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = e0 + r16 + 16 * i;
      v[i] = e < E ? lt[tl[h] * RG_LT + r16 + 16 * i] : -INFINITY;
      mm = fmaxf(mm, v[i]);
    }
    m[h] = row16_max(mm);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = e0 + r16 + 16 * i;
      ss += e < E ? __expf(v[i] - m[h]) : 0.f;
      key[h][i] = e < E ? topk_key(v[i], e) : 0ull;
    }
    sm[h] = row16_sum(ss);
  }
  row16_topk_keys2(key, rp.topk, kl + tl[0] * 16, kl + tl[1] * 16);
  dma::bar_lds();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = t0 + tl[h];
    if (t < T) {
      const size_t at = (size_t)t * ny + y;
      if (r16 < rp.topk) rp.keys[at * rp.topk + r16] = kl[tl[h] * 16 + r16];
      if (r16 == 0) {
        rp.stat[2 * at] = m[h];
        rp.stat[2 * at + 1] = sm[h];
      }
    }
  }
}

template <int EPL>
__global__ __launch_bounds__(256) void route_softmax_kernel(
    float* logits, float* __restrict__ w_out, int* __restrict__ id_out, int T,
    int E, int topk, float eps, int ks, float* __restrict__ gate,
    int* __restrict__ chunk_hist, ActQuant aq, const float* __restrict__ bias) {
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  // the token's activation row as well (prefill: in place of the
  // activation-quant launch; C2 routing 11.8 + quant 11.3 -> 19.8 us)
  if (aq.x) act_quant_row(aq.x, t, aq.H, aq.pow2, aq.q, aq.s, aq.gate_w, aq.gate_out);
  route_softmax_token<EPL>(logits + (size_t)t * E, ks, (long)T * E, E, topk, eps,
                           w_out + (size_t)t * topk, id_out + (size_t)t * topk,
                           nullptr, bias);
  if (gate && lane == 0) route_gate_finish(gate, T, t, ks);
  if (chunk_hist && lane < topk) {  // lane reads back its own id
    const int a = t * topk + lane;
    atomicAdd(&chunk_hist[(size_t)(a / PERM_CHUNK) * E + id_out[a]], 1);
  }
}

// The fused prefill router's second launch: token t's routing from the
// tiles' partials (RouterPart, ny tiles). The ny * topk candidate keys
// (at most 64 EPL) go one per lane slot; their top-k is the top-k of the
// whole logits row, as every expert outside a tile's top-k has topk
// larger keys in its own tile. The softmax normaliser is
// M = max m_y, S = sum over y in order of s_y exp(m_y - M).
template <int EPL>
__global__ __launch_bounds__(256) void route_merge_kernel(
    RouterPart rp, int ny, float* __restrict__ w_out, int* __restrict__ id_out,
    int T, int E, float eps, int* __restrict__ chunk_hist) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  const int topk = rp.topk, nk = ny * topk;
  const uint64_t* kr = rp.keys + (size_t)t * nk;
  uint64_t key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int j = lane + 64 * i;
    key[i] = j < nk ? kr[j] : 0ull;
  }
  const float* sr = rp.stat + (size_t)t * ny * 2;
  float m = -INFINITY;
  for (int y = 0; y < ny; ++y) m = fmaxf(m, sr[2 * y]);
  float s = 0.f;
  for (int y = 0; y < ny; ++y) s += sr[2 * y + 1] * expf(sr[2 * y] - m);
  const uint64_t pick = wave_topk_keys<EPL>(key, topk);
  softmax_emit(pick, m, s, topk, eps, w_out + (size_t)t * topk,
               id_out + (size_t)t * topk, nullptr);
  // every pick is an expert (the tiles hold at least topk candidates, as
  // E >= topk); the range check keeps a damaged partial from indexing out
  const int id = topk_key_id(pick);
  if (chunk_hist && lane < topk && (unsigned)id < (unsigned)E) {
    const int a = t * topk + lane;
    atomicAdd(&chunk_hist[(size_t)(a / PERM_CHUNK) * E + id], 1);
  }
}

// Descending top-k (topk <= 16) of one token's keys per 16-lane row (N per
// lane, 0 = none, distinct), as row16_topk_keys2 for a single token: pick
// j goes to kl[j].
template <int N>
__device__ __forceinline__ void row16_topk_into(uint64_t (&key)[N], int topk,
                                                uint64_t* kl) {
  sort_desc<N>(key);
  for (int kk = 0; kk < topk; ++kk) {
    const uint32_t hi = (uint32_t)(key[0] >> 32);
    bool own = hi == row16_max_u32(hi);
    if (__popcll(__ballot(own)) != 4) {
      const uint32_t mlo = row16_max_u32(own ? (uint32_t)key[0] : 0u);
      own = own && (uint32_t)key[0] == mlo;
    }
    if (own) {
      kl[kk] = key[0];
#pragma unroll
      for (int i = 0; i + 1 < N; ++i) key[i] = key[i + 1];
      key[N - 1] = 0;
    }
  }
}

// route_merge_kernel for ny * topk <= 128 candidates: a 16-lane row per
// token (KPL keys per lane), 16 tokens per workgroup; a pick is a row
// reduction of four DPP steps rather than a wave's six, and one wave
// instruction serves four tokens. Rows past T run on token T - 1 (the
// picks' ballot counts the wave's four rows) and write nothing. The
// picks' probabilities are added over the row (lanes past topk add 0).
template <int KPL>
__global__ __launch_bounds__(256) void route_merge_row_kernel(
    RouterPart rp, int ny, float* __restrict__ w_out, int* __restrict__ id_out,
    int T, int E, float eps, int* __restrict__ chunk_hist) {
  __shared__ uint64_t kl[16][16];
  const int r16 = threadIdx.x & 15, slot = threadIdx.x >> 4;
  const int t_raw = blockIdx.x * 16 + slot;
  const bool live = t_raw < T;
  const int t = live ? t_raw : T - 1;
  const int topk = rp.topk, nk = ny * topk;
  const uint64_t* kr = rp.keys + (size_t)t * nk;
  uint64_t key[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int j = r16 + 16 * i;
    key[i] = j < nk ? kr[j] : 0ull;
  }
  const float* sr = rp.stat + (size_t)t * ny * 2;
  float m = -INFINITY;
  for (int y = 0; y < ny; ++y) m = fmaxf(m, sr[2 * y]);
  float s = 0.f;
  for (int y = 0; y < ny; ++y) s += sr[2 * y + 1] * expf(sr[2 * y] - m);
  row16_topk_into<KPL>(key, topk, kl[slot]);
  __syncthreads();
  const uint64_t pick = r16 < topk ? kl[slot][r16] : 0ull;
  const float pn = r16 < topk ? expf(topk_key_value(pick) - m) / s : 0.f;
  const float wsum = row16_sum(pn);
  const int id = topk_key_id(pick);
  if (live && r16 < topk) {
    w_out[(size_t)t * topk + r16] = pn / (wsum + eps);
    id_out[(size_t)t * topk + r16] = id;
    // every pick is an expert (E >= topk); the range check keeps a damaged
    // partial from indexing out
    if (chunk_hist && (unsigned)id < (unsigned)E) {
      const int a = t * topk + r16;
      atomicAdd(&chunk_hist[(size_t)(a / PERM_CHUNK) * E + id], 1);
    }
  }
}

// Decode (T * topk <= PERM_FUSED_MAX_N, E <= PERM_FUSED_MAX_E): softmax
// top-k of every token (wave w takes tokens w, w + 16, ...) and the
// expert-major permutation in one workgroup, the ids passed through LDS.
template <int EPL>
__global__ __launch_bounds__(1024) void route_permute_small_kernel(
    float* logits, float* __restrict__ w_out, int* __restrict__ id_out, int T,
    int E, int topk, float eps, int nbits, int bm, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ sorted_idx,
    int* __restrict__ inv_pos, int* __restrict__ tile_info,
    int* __restrict__ num_tiles, int max_tiles, int ks,
    float* __restrict__ gate, int* __restrict__ zero, int nzero,
    const float* __restrict__ bias) {
  __shared__ int hist[PERM_FUSED_WAVES][PERM_FUSED_MAX_E];
  __shared__ int sh[1024];
  __shared__ int ids_lds[PERM_FUSED_MAX_N];
  const int wave = threadIdx.x >> 6;
  for (int t = wave; t < T; t += PERM_FUSED_WAVES) {
    // fewer slice loads in flight: 16 waves share the register file
    route_softmax_token<EPL, (EPL >= 32 ? 1 : (32 / EPL < 8 ? 32 / EPL : 8))>(
        logits + (size_t)t * E, ks, (long)T * E, E, topk, eps,
        w_out + (size_t)t * topk, id_out + (size_t)t * topk, ids_lds + t * topk,
        bias);
    if (gate && (threadIdx.x & 63) == 0) route_gate_finish(gate, T, t, ks);
  }
  __syncthreads();
  permute_fused_body(ids_lds, T * topk, E, nbits, bm, counts, offsets,
                     sorted_idx, inv_pos, tile_info, num_tiles, max_tiles,
                     hist, sh, zero, nzero);
}

// Scored routing with selection bias and optional group limit
// (ref/deepseek_v4.py:522-561; group limit per DeepSeek-V3 noaux_tc): one
// token per wave (route_grouped_token).
template <int EPL>
__global__ __launch_bounds__(256) void route_grouped_kernel(
    float* logits, const float* __restrict__ bias, float* __restrict__ w_out,
    int* __restrict__ id_out, int T, int E, int topk, int n_group,
    int topk_group, int scoring, float route_scale, int ks) {
  __shared__ float sb[4][EPL * 64];
  __shared__ float scl[4][EPL * 64];
  const int wv = threadIdx.x >> 6;
  const int t_raw = blockIdx.x * (blockDim.x >> 6) + wv;
  const bool active = t_raw < T;
  const int t = active ? t_raw : T - 1;  // idle waves mirror the last row
  // waves past T mirror row T - 1 without writing it
  route_grouped_token<EPL>(logits + (size_t)t * E, ks, (long)T * E, active, E,
                           topk, n_group, topk_group, scoring, route_scale,
                           bias, sb[wv], scl[wv],
                           active ? w_out + (size_t)t * topk : nullptr,
                           active ? id_out + (size_t)t * topk : nullptr,
                           nullptr);
}

// Hash layers (ref/deepseek_v4.py:545-552; upstream model.py:620-627,
// text branch): the expert ids of token t are tid2eid[clip(token_ids[t],
// 0, vocab - 1)] in table order -- no bias, no top-k -- and the weights are
// those experts' scores, renormalized unless softmax (summed in slot
// order), times route_scale. One wave per token; the row's scores go
// through LDS so that lane j can read the score of its slot's expert.
template <int EPL>
__global__ __launch_bounds__(256) void route_hash_kernel(
    float* logits, const int* __restrict__ token_ids,
    const int* __restrict__ tid2eid, int vocab, float* __restrict__ w_out,
    int* __restrict__ id_out, int T, int E, int topk, int scoring,
    float route_scale, int ks) {
  __shared__ float sb[4][EPL * 64];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int t_raw = blockIdx.x * (blockDim.x >> 6) + wv;
  const bool active = t_raw < T;
  const int t = active ? t_raw : T - 1;
  float sc[EPL];
  // waves past T mirror row T - 1 without writing it
  gate_scores_row<EPL>(logits + (size_t)t * E, ks, (long)T * E, active, E,
                       scoring, sc);
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (lane + 64 * i < E) sb[wv][lane + 64 * i] = sc[i];
  __syncthreads();
  const int tok = min(max(token_ids[t], 0), vocab - 1);
  int e = 0;
  float se = 0.f;
  if (lane < topk) {
    e = tid2eid[(size_t)tok * topk + lane];
    se = (e >= 0 && e < E) ? sb[wv][e] : __uint_as_float(0x7FC00000u);
  }
  float wsum = 0.f;
  for (int j = 0; j < topk; ++j) wsum += __shfl(se, j, kWave);
  if (active && lane < topk) {
    const float wv_ = scoring == SCORE_SOFTMAX ? se : se / wsum;
    w_out[(size_t)t * topk + lane] = wv_ * route_scale;
    id_out[(size_t)t * topk + lane] = e;
  }
}

static int epl_for(int E) {
  int epl = 1;
  while (epl * 64 < E) epl *= 2;
  return epl;
}

// Tokens (waves) per workgroup of the multi-workgroup routing kernels: 4,
// or 1 over split logits, whose ks slices per row are then read through T
// CUs rather than T / 4 (the reads are bound by per-CU bandwidth).
static int route_tokens_per_block(int ks) { return ks > 1 ? 1 : 4; }

// K chunks of the decode router: at least two, and enough that each of a
// workgroup's 8 waves takes at most four 32-wide K slices, one round of
// loads in flight together. H = 2048 (C3): 2, as every further slice costs
// the routing about what the router saves (C3 B=32, layer: unsplit
// 155-157 us, 2 chunks 153-155, 4 chunks 153-156, 8 chunks 156-157).
// H = 7168 (C4): 7; two chunks left each wave four rounds of loads (the
// router 8.9 us at B=1), and 8 chunks took C4 decode B=1 / 8 / 32 from
// 98 / 281 / 680 to 94 / 274 / 672 us.
int router_ksplit(int T, int H) {
  if (T > RG_SMALL_T) return 1;
  const int one_round = (H / 32 + 31) / 32;
  return std::max(std::max(1, std::min(2, H / 256)), one_round);
}

static int launch_router_small(const uint16_t* x, const uint16_t* w,
                               float* logits, int T, int E, int H,
                               const uint16_t* sgl, float* gate_out, int ks,
                               hipStream_t st, int* zero = nullptr,
                               long nzero = 0) {
  SLLM_REQUIRE(ks >= 1 && ks <= H / 32, "router_small: bad K split %d", ks);
  SLLM_REQUIRE(nzero >= 0 && (nzero == 0 || zero), "router_small: bad zero range");
  const dim3 grid(ceil_div(E, 16) + (gate_out ? 1 : 0), ks);
#define CASE(n)                                                              \
  router_gemm_small_kernel<n><<<grid, 512, 0, st>>>(x, w, logits, T, E, H,   \
                                                    sgl, gate_out, zero, nzero)
  switch (ceil_div(T, 16)) {
    case 1: CASE(1); break;
    case 2: CASE(2); break;
    case 3: CASE(3); break;
    default: CASE(4); break;
  }
#undef CASE
  SLLM_LAUNCHED();
  return 0;
}

int launch_router_gemm(const uint16_t* x, const uint16_t* w, float* logits,
                       int T, int E, int H, hipStream_t st, int ks,
                       int* zero, long zero_n) {
  SLLM_REQUIRE(x && w && logits, "router_gemm: null pointer");
  SLLM_REQUIRE(T > 0 && E > 0 && H > 0 && H % 128 == 0,
               "router_gemm: need T,E>0 and H %% 128 == 0 (T=%d E=%d H=%d)",
               T, E, H);
  SLLM_REQUIRE(ks == 1 || T <= RG_SMALL_T, "router_gemm: K split needs T <= %d",
               RG_SMALL_T);
  SLLM_REQUIRE(zero_n == 0 || (zero && T > RG_SMALL_T),
               "router_gemm: zeroing needs the prefill kernel");
  if (T <= RG_SMALL_T) {
    return launch_router_small(x, w, logits, T, E, H, nullptr, nullptr, ks, st);
  } else {
    dim3 grid(ceil_div(T, RG_TT), ceil_div(E, RG_TE));
    router_gemm_kernel<<<grid, 512, 0, st>>>(x, w, logits, T, E, H, zero,
                                             zero_n);
  }
  SLLM_LAUNCHED();
  return 0;
}

static bool topk_ok(int E, int topk) {
  return E > 0 && topk > 0 && topk <= 16 && topk <= E &&
         (long)ceil_div(E, RG_TE) * topk <= 512;
}

// 1-D grid of router_topk_kernel: ceil(E / 128) expert tiles for each of
// the ceil(T / 64) token tiles, rounded up to whole rounds of 8 (one token
// tile per XCD slot).
static unsigned router_topk_grid(int T, int E) {
  return (unsigned)(8 * ceil_div(ceil_div(T, RG_TT), 8) * ceil_div(E, RG_TE));
}

bool router_topk_fits(int T, int E, int topk, int H) {
  return T > RG_SMALL_T && topk_ok(E, topk) && H > 0 && H % RG_KC == 0 &&
         H <= RT_GATE_MAX;
}

size_t router_part_bytes(int T, int E, int topk) {
  const size_t n = (size_t)T * ceil_div(E, RG_TE);
  return n * 8 + n * topk * 8;
}

RouterPart router_part_at(char* base, int T, int E, int topk) {
  const size_t n = (size_t)T * ceil_div(E, RG_TE);
  RouterPart rp{};
  rp.stat = (float*)base;
  rp.keys = (uint64_t*)(base + n * 8);
  rp.topk = topk;
  return rp;
}

int launch_router_topk(const uint16_t* x, const uint16_t* w, float* logits,
                       int T, int E, int H, const RouterPart& rp,
                       hipStream_t st, int* zero, long zero_n) {
  SLLM_REQUIRE(x && w && rp.stat && rp.keys, "router_topk: null pointer");
  SLLM_REQUIRE(router_topk_fits(T, E, rp.topk, H),
               "router_topk: need T > %d, H %% 128 == 0, H <= %d, topk <= 16, "
               "ceil(E / 128) * topk <= 512 (T=%d E=%d H=%d k=%d)",
               RG_SMALL_T, RT_GATE_MAX, T, E, H, rp.topk);
  SLLM_REQUIRE(!rp.q || rp.s, "router_topk: quantized rows without scales");
  SLLM_REQUIRE(!rp.gate_w || (rp.q && rp.gate_out),
               "router_topk: gate needs the quantization and gate buffers");
  SLLM_REQUIRE(zero_n == 0 || zero, "router_topk: null zero range");
  router_topk_kernel<<<router_topk_grid(T, E), 512, 0, st>>>(x, w, logits, T, E, H, zero,
                                           zero_n, rp);
  SLLM_LAUNCHED();
  return 0;
}

bool router_logits_quant_fits(int T, int H) {
  return T > RG_SMALL_T && H > 0 && H % RG_KC == 0;
}

int launch_router_logits_quant(const uint16_t* x, const uint16_t* w,
                               float* logits, int T, int E, int H, uint8_t* q,
                               float* s, int pow2, hipStream_t st) {
  SLLM_REQUIRE(x && w && logits && q && s, "router_logits_quant: null pointer");
  SLLM_REQUIRE(E > 0 && router_logits_quant_fits(T, H),
               "router_logits_quant: need T > %d, H %% 128 == 0 (T=%d E=%d H=%d)",
               RG_SMALL_T, T, E, H);
  RouterPart rp{};
  rp.q = q;
  rp.s = s;
  rp.pow2 = pow2 ? 1 : 0;
  router_topk_kernel<<<router_topk_grid(T, E), 512, 0, st>>>(x, w, logits, T, E, H,
                                                             nullptr, 0, rp);
  SLLM_LAUNCHED();
  return 0;
}

int launch_route_merge(const RouterPart& rp, int T, int E, float eps,
                       float* w, int* ids, hipStream_t st, int* chunk_hist) {
  SLLM_REQUIRE(rp.stat && rp.keys && w && ids, "route_merge: null pointer");
  SLLM_REQUIRE(T > RG_SMALL_T && topk_ok(E, rp.topk),
               "route_merge: bad sizes (T=%d E=%d k=%d)", T, E, rp.topk);
  const int ny = ceil_div(E, RG_TE), nk = ny * rp.topk;
  if (nk <= 128) {
    const int kpl = nk <= 16 ? 1 : nk <= 32 ? 2 : nk <= 64 ? 4 : 8;
    dim3 grid(ceil_div(T, 16));
    switch (kpl) {
#define CASE(n)                                                               \
  case n:                                                                     \
    route_merge_row_kernel<n><<<grid, 256, 0, st>>>(rp, ny, w, ids, T, E,     \
                                                    eps, chunk_hist);         \
    break;
      CASE(1) CASE(2) CASE(4) CASE(8)
#undef CASE
    }
    SLLM_LAUNCHED();
    return 0;
  }
  dim3 grid(ceil_div(T, 4));
  switch (epl_for(nk)) {
#define CASE(n)                                                               \
  case n:                                                                     \
    route_merge_kernel<n><<<grid, 256, 0, st>>>(rp, ny, w, ids, T, E, eps,    \
                                                chunk_hist);                  \
    break;
    CASE(1) CASE(2) CASE(4) CASE(8)
#undef CASE
  }
  SLLM_LAUNCHED();
  return 0;
}

int launch_router_small_gate(const uint16_t* x, const uint16_t* w,
                             float* logits, int T, int E, int H,
                             const uint16_t* sgl, float* gate_out,
                             hipStream_t st, int ks, int* zero, long nzero) {
  SLLM_REQUIRE(x && w && logits && T > 0 && T <= RG_SMALL_T && E > 0 &&
                   H % 32 == 0 && (!gate_out || sgl),
               "router_small_gate: bad args (T=%d E=%d H=%d)", T, E, H);
  return launch_router_small(x, w, logits, T, E, H, sgl, gate_out, ks, st,
                             zero, nzero);
}

// One workgroup routes every token (a wave per token): worth it only while
// the tokens fit one pass of the 16 waves; larger batches route with the
// multi-workgroup kernel.
bool route_inline_fits(int T, int E, int topk, long max_tiles) {
  return T > 0 && T <= RG_SMALL_T && E >= topk && E <= RI_MAX_E &&
         topk > 0 && topk <= 64 && (long)T * topk <= RI_MAX_N &&
         max_tiles <= RI_MAX_TILES;
}

bool route_permute_small_fits(int T, int E, int topk) {
  return T <= PERM_FUSED_WAVES && (long)T * topk <= PERM_FUSED_MAX_N &&
         E <= PERM_FUSED_MAX_E;
}

int launch_route_permute_small(const float* logits, float* w, int* ids, int T,
                               int E, int topk, float eps, int bm,
                               int* counts, int* offsets, int* sorted_idx,
                               int* inv_pos, int* tile_info, int* num_tiles,
                               int max_tiles, hipStream_t st, int ks,
                               float* gate, int* zero, int nzero,
                               const float* bias) {
  SLLM_REQUIRE(ks >= 1 && (!gate || ks > 1),
               "route_permute_small: bad logit slices %d", ks);
  SLLM_REQUIRE(nzero == 0 || (zero && nzero > 0), "route_permute_small: bad zero range");
  SLLM_REQUIRE(logits && w && ids && route_permute_small_fits(T, E, topk) &&
                   topk > 0 && topk <= E && topk <= 64 && T > 0,
               "route_permute_small: bad sizes (T=%d E=%d k=%d)", T, E, topk);
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  switch (epl_for(E)) {
#define CASE(n)                                                               \
  case n:                                                                     \
    route_permute_small_kernel<n><<<1, 1024, 0, st>>>(                        \
        (float*)logits, w, ids, T, E, topk, eps, nbits, bm, counts, offsets,  \
        sorted_idx, inv_pos, tile_info, num_tiles, max_tiles, ks, gate,      \
        zero, nzero, bias);                                                   \
    break;
    CASE(1) CASE(2) CASE(4) CASE(8) CASE(16)
#undef CASE
    default:
      SLLM_REQUIRE(false, "route_permute_small: E=%d too large", E);
  }
  SLLM_LAUNCHED();
  return 0;
}

int launch_route_softmax(const float* logits, float* w, int* ids, int T,
                         int E, int topk, float eps, hipStream_t st, int ks,
                         float* gate, int* chunk_hist, const ActQuant* aq_in,
                         const float* bias) {
  SLLM_REQUIRE(logits && w && ids && ks >= 1 && (!gate || ks > 1),
               "route_softmax: null pointer or bad logit slices");
  ActQuant aq{};
  if (aq_in && aq_in->x) {
    aq = *aq_in;
    SLLM_REQUIRE(aq.q && aq.s && aq.H > 0 && aq.H % 128 == 0 &&
                     (!aq.gate_w || aq.gate_out),
                 "route_softmax: bad activation-quant arguments (H=%d)", aq.H);
  }
  SLLM_REQUIRE(T > 0 && E > 0 && topk > 0 && topk <= E && E <= 2048 &&
                   topk <= 64,
               "route_softmax: need 0<topk<=E<=2048, topk<=64 (E=%d k=%d)",
               E, topk);
  const int tpb = route_tokens_per_block(ks);
  dim3 grid(ceil_div(T, tpb));
  switch (epl_for(E)) {
#define CASE(n)                                                               \
  case n:                                                                     \
    route_softmax_kernel<n><<<grid, 64 * tpb, 0, st>>>(                       \
        (float*)logits, w, ids, T, E, topk, eps, ks, gate, chunk_hist, aq,    \
        bias);                                                                \
    break;
    CASE(1) CASE(2) CASE(4) CASE(8) CASE(16) CASE(32)
#undef CASE
  }
  SLLM_LAUNCHED();
  return 0;
}

int launch_route_grouped(const float* logits, const float* bias, float* w,
                         int* ids, int T, int E, int topk, int n_group,
                         int topk_group, int scoring, float route_scale,
                         hipStream_t st, int ks) {
  SLLM_REQUIRE(logits && w && ids && ks >= 1, "route_grouped: null pointer");
  SLLM_REQUIRE(T > 0 && E > 0 && topk > 0 && topk <= E && E <= 2048 &&
                   topk <= 64,
               "route_grouped: need 0<topk<=E<=2048, topk<=64");
  SLLM_REQUIRE(scoring >= 0 && scoring <= 2, "route_grouped: bad scoring %d",
               scoring);
  if (n_group > 1) {
    SLLM_REQUIRE(n_group <= 64 && E % n_group == 0 && topk_group >= 1 &&
                     topk_group <= n_group &&
                     topk_group * (E / n_group) >= topk,
                 "route_grouped: bad group config (E=%d G=%d kg=%d k=%d)", E,
                 n_group, topk_group, topk);
  }
  const int tpb = route_tokens_per_block(ks);
  dim3 grid(ceil_div(T, tpb));
  switch (epl_for(E)) {
#define CASE(n)                                                               \
  case n:                                                                     \
    route_grouped_kernel<n><<<grid, 64 * tpb, 0, st>>>(                       \
        (float*)logits, bias, w, ids, T, E, topk, n_group, topk_group,        \
        scoring, route_scale, ks);                                            \
    break;
    CASE(1) CASE(2) CASE(4) CASE(8) CASE(16) CASE(32)
#undef CASE
  }
  SLLM_LAUNCHED();
  return 0;
}

int launch_route_hash(const float* logits, const int* token_ids,
                      const int* tid2eid, int vocab, float* w, int* ids,
                      int T, int E, int topk, int scoring, float route_scale,
                      hipStream_t st, int ks) {
  SLLM_REQUIRE(logits && token_ids && tid2eid && w && ids && ks >= 1,
               "route_hash: null pointer");
  SLLM_REQUIRE(T > 0 && E > 0 && E <= 2048 && topk > 0 && topk <= 64 &&
                   topk <= E && vocab > 0 && scoring >= 0 && scoring <= 2,
               "route_hash: bad sizes (T=%d E=%d k=%d vocab=%d scoring=%d)",
               T, E, topk, vocab, scoring);
  const int tpb = route_tokens_per_block(ks);
  const int grid = ceil_div(T, tpb);
  switch (epl_for(E)) {
#define CASE(n)                                                               \
  case n:                                                                     \
    route_hash_kernel<n><<<grid, 64 * tpb, 0, st>>>((float*)logits, token_ids, \
                                               tid2eid, vocab, w, ids, T, E,  \
                                               topk, scoring, route_scale,    \
                                               ks);                           \
    break;
    CASE(1) CASE(2) CASE(4) CASE(8) CASE(16) CASE(32)
#undef CASE
    default:
      SLLM_REQUIRE(false, "route_hash: E=%d too large", E);
  }
  SLLM_LAUNCHED();
  return 0;
}

}  // namespace sllm

using namespace sllm;

extern "C" {

// ref: kernels/cuda/qwen4.cu:279-298 (host-pointer variant).
int sllm_q4_moe_router(const float* logits, float* w_out, int* id_out, int n,
                       int E, int topk) {
  if (n <= 0 || E <= 0 || topk <= 0 || topk > E || E > 2048 || topk > 16) {
    set_error("sllm_q4_moe_router: bad args (n=%d E=%d topk=%d)", n, E, topk);
    return -1;
  }
  float *dl = nullptr, *dw = nullptr;
  int* di = nullptr;
  int rc = -1;
  if (hipMalloc(&dl, (size_t)n * E * sizeof(float)) != hipSuccess ||
      hipMalloc(&dw, (size_t)n * topk * sizeof(float)) != hipSuccess ||
      hipMalloc(&di, (size_t)n * topk * sizeof(int)) != hipSuccess) {
    set_error("sllm_q4_moe_router: hipMalloc failed");
  } else if (hipMemcpy(dl, logits, (size_t)n * E * sizeof(float),
                       hipMemcpyHostToDevice) != hipSuccess) {
    set_error("sllm_q4_moe_router: H2D failed");
  } else if (launch_route_softmax(dl, dw, di, n, E, topk, 1e-20f, 0) == 0 &&
             hipMemcpy(w_out, dw, (size_t)n * topk * sizeof(float),
                       hipMemcpyDeviceToHost) == hipSuccess &&
             hipMemcpy(id_out, di, (size_t)n * topk * sizeof(int),
                       hipMemcpyDeviceToHost) == hipSuccess) {
    rc = 0;
  } else if (last_error()[0] == 0) {
    set_error("sllm_q4_moe_router: D2H failed");
  }
  (void)hipFree(dl);
  (void)hipFree(dw);
  (void)hipFree(di);
  return rc;
}

// ref: kernels/cuda/qwen4.cu:785-793 (device-pointer variant, no sync).
int sllm_q4_moe_router_dev(const float* logits, float* w_out, int* id_out,
                           int n, int E, int topk) {
  if (n <= 0 || E <= 0 || topk <= 0 || topk > E || E > 2048 || topk > 16) {
    set_error("sllm_q4_moe_router_dev: bad args (n=%d E=%d topk=%d)", n, E,
              topk);
    return -1;
  }
  return launch_route_softmax(logits, w_out, id_out, n, E, topk, 1e-20f, 0);
}

int sllm_moe_router_gemm(const void* x_bf16, const void* w_bf16,
                         float* logits, int T, int E, int H, void* stream) {
  return launch_router_gemm((const uint16_t*)x_bf16, (const uint16_t*)w_bf16,
                            logits, T, E, H, (hipStream_t)stream);
}

int sllm_moe_route_softmax(const float* logits, float* w_out, int* id_out,
                           int T, int E, int topk, float eps, void* stream) {
  return launch_route_softmax(logits, w_out, id_out, T, E, topk, eps,
                              (hipStream_t)stream);
}

int sllm_moe_route_hash(const float* logits, const int* token_ids,
                        const int* tid2eid, int vocab, float* w_out,
                        int* id_out, int T, int E, int topk, int scoring,
                        float route_scale, void* stream) {
  return launch_route_hash(logits, token_ids, tid2eid, vocab, w_out, id_out,
                           T, E, topk, scoring, route_scale,
                           (hipStream_t)stream);
}

int sllm_moe_route_grouped(const float* logits, const float* bias,
                           float* w_out, int* id_out, int T, int E, int topk,
                           int n_group, int topk_group, int scoring,
                           float route_scale, void* stream) {
  return launch_route_grouped(logits, bias, w_out, id_out, T, E, topk,
                              n_group, topk_group, scoring, route_scale,
                              (hipStream_t)stream);
}

}  // extern "C"
