// Compute-dense grouped expert GEMM over packed FP8 weights, for prefill
// launches whose experts average more than one 128-row tile: a skewed
// Qwen-style layer (C5: hot experts with tens of tiles) and the shared
// expert of a DeepSeek-style layer (every token one row, 64 tiles at 8192
// tokens), which the streaming kernel runs at a third of the matrix cores'
// rate (its activation fragments feed two MFMAs each).
//
// The structure of the MXFP4 dense kernel (gemm_dense.hip) with the FP8
// weight layout of the streaming kernel (gemm_stream.hip), same items and
// the same arithmetic in the same order, so the outputs agree with the
// streaming kernel's bit for bit:
// * An item is a 128-row tile x one packed slab (gate/up: 128 h columns,
//   the gate and up columns of each; down: 256 output columns); K steps of
//   128. Wave w = 4 r + c computes rows [64 r, +64) x the slab's packed
//   waves 2 c, 2 c + 1 (subtiles g, u, g, u or four 16-column ones): 64
//   accumulators, each activation fragment feeding four MFMAs.
// * Operands staged in LDS by direct-to-LDS loads, three stages two steps
//   ahead: the step's 128 gathered activation rows (XOR-swizzled by row),
//   its 32 KB packed weight block verbatim (already in MFMA fragment order)
//   and the rows' activation scales. Waves 0-3 issue them (thirteen loads
//   per wave per stage), spread over their first groups' MFMAs (on an
//   item's last step too, before its epilogue); the next
//   stage is made ready (vmcnt, then a fence-free barrier) before a step's
//   last group, whose MFMA issue covers the barrier and the next step's
//   first fragment reads.
// * Block scales. fp32 (C5, the reference's FP8 layout): each 16x16x128
//   MFMA yields the unscaled partial of one K step, added as
//   acc += partial * (s_x[row] * s_w) as the streaming kernel does, the
//   partials of group mi rescaled while group mi + 1's MFMAs run. Power of
//   two (pow2 activation scales and weight scales, the DeepSeek shared
//   expert): the MFMA applies both as e8m0 scales. The weight scales of an
//   item's K steps are read once into LDS with its row tables.
#include <type_traits>

#include "launch.h"
#include "lds_dma.h"

namespace sllm {

namespace {

using namespace dma;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int D8_BM = 128;                    // rows per tile
constexpr int D8_THREADS = 512;               // eight waves
constexpr int D8_STAGES = 3;
constexpr int D8_ITEMS = 4;                   // items per chunk (LDS tables)
constexpr int D8_KBMAX = 64;                  // K steps in the scale table
constexpr int D8_A = D8_BM * 128;             // activations: rows x 128 e4m3
constexpr int D8_B = 32768;                   // packed fp8 block (slab, K step)
constexpr int D8_SX = D8_BM * 4;              // activation scales (fp32)
constexpr int D8_STAGE = D8_A + D8_B + D8_SX;
constexpr int D8_LOADS = 13;                  // per loader wave per stage

template <int MODE, bool F32S>
__global__ __launch_bounds__(D8_THREADS, 1) void moe_dense8_kernel(
    SegDesc S, int topk, float limit, int pow2) {
  // three stages as three arrays: the compiler then sees that a step's LDS
  // reads (one stage) do not alias the loads in flight (the other two)
  __shared__ __attribute__((aligned(16))) uint8_t stg0[D8_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stg1[D8_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stg2[D8_STAGE];
  __shared__ int4 desc[D8_ITEMS];
  __shared__ int rsrc[D8_ITEMS][D8_BM];
  __shared__ float rwl[D8_ITEMS][D8_BM];        // row weights (1 without row_w)
  __shared__ float wsc[D8_ITEMS][D8_KBMAX][2];  // weight scales per K step
  __shared__ float red[D8_BM][4];               // gate/up: row amax per column wave

  constexpr int NTW = MODE == 0 ? 128 : 256;  // h / output columns per item
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4, lc = lane & 15;
  const int wr = wave >> 2, wc = wave & 3;
  const int K = S.K, KB = K / 128, N = S.N;
  const int ntn = N / NTW;  // packed slabs across N (items per row tile)

  const int rtiles = S.tile_info ? *S.num_tiles : (S.total_rows + D8_BM - 1) / D8_BM;
  const int total = rtiles * ntn;
  const int nx = gridDim.x / 8;
  const int xcd = blockIdx.x % 8, jx = blockIdx.x / 8;
  const int xbeg = (int)((long)total * xcd / 8);
  const int xend = (int)((long)total * (xcd + 1) / 8);
  const int nall = xend - xbeg > jx ? (xend - xbeg - jx + nx - 1) / nx : 0;

  for (int cbase = 0; cbase < nall; cbase += D8_ITEMS) {
    const int nitems = min(D8_ITEMS, nall - cbase);
    if (tid < nitems) {
      const int it = xbeg + jx + (cbase + tid) * nx;
      const int rt = it / ntn, np = it % ntn;
      if (S.tile_info) {
        const int4 d = *(const int4*)(S.tile_info + 4 * rt);
        desc[tid] = make_int4(np, d.x, d.y, min(D8_BM, d.z));
      } else {
        desc[tid] = make_int4(np, 0, rt * D8_BM, min(D8_BM, S.total_rows - rt * D8_BM));
      }
    }
    __syncthreads();
    for (int q = tid; q < nitems * D8_BM; q += D8_THREADS) {
      const int i = q / D8_BM, r = q % D8_BM;
      const int4 d = desc[i];
      const int p = d.z + (r < d.w ? r : 0);  // rows past the tile read row 0
      rsrc[i][r] = S.gather ? S.sorted_idx[p] / topk : p;
      rwl[i][r] = S.row_w ? S.row_w[S.row_w_by_idx ? S.sorted_idx[p] : p] : 1.f;
    }
    // weight scales (reference layout): gate/up [e][slab][kb] of W1 and W3;
    // down [e][128-column block][kb], the slab's two blocks
    for (int q = tid; q < nitems * KB * 2; q += D8_THREADS) {
      const int i = q / (KB * 2), kb = (q / 2) % KB, h = q & 1;
      const int4 d = desc[i];
      float v;
      if constexpr (MODE == 0)
        v = ((const float*)(h ? S.s1 : S.s0))[((size_t)d.y * ntn + d.x) * KB + kb];
      else
        v = ((const float*)S.s0)[((size_t)d.y * (N / 128) + 2 * d.x + h) * KB + kb];
      wsc[i][kb][h] = v;
    }
    __syncthreads();
    const int total_steps = nitems * KB;

    // ---- prefetch cursor (loader waves 0-3): activation slots
    // 256 L + 64 q + lane of the stage's 1024 16-byte chunks (slot g holds
    // chunk (g % 8) ^ (row % 8) of row g / 8), the weight block's 1 KB
    // chunks [8 L, 8 L + 8), the activation scales of rows 32 L + lane
    const bool loader = wave < 4;
    int pi = 0, pkb = 0;
    uint32_t poff[4], psx = 0;  // byte offsets from S.a / S.sa
    const uint8_t* pbw = nullptr;
    auto p_enter = [&](int i) __attribute__((always_inline)) {
      const int4 d = desc[i];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int g = 256 * wave + 64 * q + lane, row = g >> 3;
        poff[q] = (uint32_t)rsrc[i][row] * K + (((g & 7) ^ (row & 7)) << 4);
      }
      psx = (uint32_t)rsrc[i][32 * wave + (lane & 31)] * KB * 4;
      const int e = __builtin_amdgcn_readfirstlane(d.y);
      const int np = __builtin_amdgcn_readfirstlane(d.x);
      pbw = S.wp + ((size_t)e * ntn + np) * KB * D8_B + wave * 8192;
    };
    // load j of the loader's stage (a compile-time constant once unrolled):
    // 0-3 activation chunks, 4-11 weight chunks, 12 activation scales
    auto dma = [&](int j, uint8_t* base) __attribute__((always_inline)) {
      if (j < 4) {
        to_lds(S.a + poff[j] + pkb * 128, base + wave * 4096 + j * 1024, 16);
      } else if (j < 12) {
        to_lds(pbw + (size_t)pkb * D8_B + (j - 4) * 1024 + lane * 16,
               base + D8_A + wave * 8192 + (j - 4) * 1024, 16);
      } else if (lane < 32) {
        to_lds((const uint8_t*)S.sa + psx + pkb * 4, base + D8_A + D8_B + wave * 128, 4);
      }
    };
    auto advance = [&]() __attribute__((always_inline)) {
      if (++pkb == KB && pi + 1 < nitems) {
        pkb = 0;
        p_enter(++pi);
      }
    };
    auto issue = [&](uint8_t* base) __attribute__((always_inline)) {
      if (!loader) return;
#pragma unroll
      for (int j = 0; j < D8_LOADS; ++j) dma(j, base);
      advance();
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[mi][q] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // ---- epilogues ----------------------------------------------------------
    // acc[mi][q][v]: row 64 wr + 16 mi + lc of the tile, column 4 lg + v of
    // subtile q (gate/up: q = 0, 2 gate and 1, 3 up of packed waves 2 wc,
    // 2 wc + 1; down: columns 64 wc + 16 q + 4 lg + v of the slab)
    auto epilogue = [&](int i) __attribute__((always_inline)) {
      const int4 d = desc[i];
      const int np = d.x, rb = d.z, rows = d.w;
      const int ngrp = min(4, max(0, (rows - 64 * wr + 15) >> 4));
      if constexpr (MODE == 0) {
        // h = silu(g) * u * route weight; per-row amax over the slab's four
        // column waves (one 128-column quantization block); e4m3 with the
        // row's scale
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          if (mi < ngrp) {
            const int t = 64 * wr + 16 * mi + lc;
            const float rw = rwl[i][t];
            float amax = 0.f;
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                float g = acc[mi][2 * pr][v], u = acc[mi][2 * pr + 1][v];
                if (limit > 0.f) {
                  u = fminf(fmaxf(u, -limit), limit);
                  g = fminf(g, limit);
                }
                const float h = silu_fast(g) * u * rw;
                acc[mi][2 * pr][v] = h;
                amax = fmaxf(amax, fabsf(h));
              }
            }
            amax = rows4_max(amax);
            if (lg == 0) red[t][wc] = amax;
          }
        }
        bar_lds();
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          if (mi < ngrp) {
            const int t = 64 * wr + 16 * mi + lc;
            const float amax = fmaxf(fmaxf(red[t][0], red[t][1]), fmaxf(red[t][2], red[t][3]));
            float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
            float inv;
            if (pow2) {
              const uint32_t bits = __float_as_uint(sc);
              const int ex = (int)((bits >> 23) & 0xFF) - 127 + ((bits & 0x7FFFFF) ? 1 : 0);
              sc = __uint_as_float((uint32_t)(ex + 127) << 23);
              inv = __uint_as_float((uint32_t)(127 - ex) << 23);
            } else {
              inv = __builtin_amdgcn_rcpf(sc);
            }
            if (t < rows) {
              uint8_t* hrow = S.hq + (size_t)(rb + t) * N + np * 128 + 32 * wc;
#pragma unroll
              for (int pr = 0; pr < 2; ++pr) {
                float y[4];
#pragma unroll
                for (int v = 0; v < 4; ++v)
                  y[v] = fminf(fmaxf(acc[mi][2 * pr][v] * inv, -448.f), 448.f);
                *(uint32_t*)(hrow + 16 * pr + lg * 4) = f32x4_to_e4m3(y[0], y[1], y[2], y[3]);
              }
              if (wc == 0 && lg == 0) S.hs[(size_t)(rb + t) * (N / 128) + np] = sc;
            }
          }
        }
      } else {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          if (mi < ngrp) {
            const int t = 64 * wr + 16 * mi + lc;
            if (t < rows) {
              const float rw = rwl[i][t];
              uint16_t* yrow = S.y + (size_t)(rb + t) * N + np * 256 + 64 * wc;
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const uint32_t lo = pk_bf16(acc[mi][q][0] * rw, acc[mi][q][1] * rw);
                const uint32_t hi = pk_bf16(acc[mi][q][2] * rw, acc[mi][q][3] * rw);
                *(uint2*)(yrow + 16 * q + lg * 4) = make_uint2(lo, hi);
              }
            }
          }
        }
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[mi][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };

    // ---- pipeline -----------------------------------------------------------
    // group mi's activation fragment and the row's scale: lane group lg
    // holds K bytes [32 lg, +32) of the step (chunks 2 lg and 2 lg + 1), the
    // K order of the packed fp8 weight fragments (fp8 x fp8 products do not
    // depend on the order, as long as both operands share it)
    struct Frag {
      v8i x;
      float sx;
    };
    auto frag_at = [&](const uint8_t* stage, int mi) __attribute__((always_inline)) {
      const int r = 64 * wr + 16 * mi + lc;
      const u32x4 x0 = *(const u32x4*)(stage + a_off(r, 2 * lg));
      const u32x4 x1 = *(const u32x4*)(stage + a_off(r, 2 * lg + 1));
      Frag f;
      f.x = (v8i){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                  (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
      f.sx = ((const float*)(stage + D8_A + D8_B))[r];
      return f;
    };
    // the step's weight fragments: subtile q = packed wave 2 wc + q / 2,
    // its (q % 2)-th 16 columns, the low and high 1 KB chunks of the block
    struct WFrag {
      v8i w0, w1, w2, w3;
    };
    auto wfrag_at = [&](const uint8_t* stage) __attribute__((always_inline)) {
      const uint8_t* B = stage + D8_A + 8 * wc * 1024 + lane * 16;
      auto one = [&](int q) __attribute__((always_inline)) {
        const u32x4 lo = *(const u32x4*)(B + 2 * q * 1024);
        const u32x4 hi = *(const u32x4*)(B + (2 * q + 1) * 1024);
        return (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                     (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      };
      WFrag g;
      g.w0 = one(0);
      g.w1 = one(1);
      g.w2 = one(2);
      g.w3 = one(3);
      return g;
    };
    auto stage_ready = [&](bool newer) __attribute__((always_inline)) {
      if (newer) wait_vm<D8_LOADS>();
      else wait_vm<0>();
      bar_lds();
    };

    Frag nf;   // the next step's first activation fragment
    WFrag ng;  // and its weight fragments
    // step s on stage J = s % 3, K step ckb of item ci (see the header)
    auto step = [&](auto J, int s, int ci, int ckb) __attribute__((always_inline)) {
      constexpr int j = decltype(J)::value;
      uint8_t* const cur = j == 0 ? stg0 : (j == 1 ? stg1 : stg2);
      uint8_t* const nst = j == 0 ? stg1 : (j == 1 ? stg2 : stg0);
      uint8_t* const nxt = j == 0 ? stg2 : (j == 1 ? stg0 : stg1);
      const bool last = ckb + 1 == KB;
      const bool spread = loader && s + 2 < total_steps;
      Frag cur_f = nf;
      const WFrag g = ng;
      // weight scale of subtile q: gate / up of the slab, or the wave's
      // 128-column block
      const float s0 = wsc[ci][ckb][MODE == 0 ? 0 : (wc >> 1)];
      const float s1 = MODE == 0 ? wsc[ci][ckb][1] : s0;
      const int ngrp = min(4, max(0, (desc[ci].w - 64 * wr + 15) >> 4));
      f32x4 part[2][4];
      auto mfmas = [&](int mi, const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const v8i wv = q == 0 ? g.w0 : (q == 1 ? g.w1 : (q == 2 ? g.w2 : g.w3));
          if constexpr (F32S) {
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            part[mi & 1][q] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wv, f.x, z, 0, 0, 0, 0, 0, 0);
          } else {
            acc[mi][q] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wv, f.x, acc[mi][q], 0, 0, 0, (int)e8m0_of((q & 1) ? s1 : s0), 0,
                (int)e8m0_of(f.sx));
          }
        }
      };
      // acc += partial * (s_x * s_w), the streaming kernel's order
      auto rescale = [&](int mi, float sx) __attribute__((always_inline)) {
        const float f0 = sx * s0, f1 = sx * s1;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float f = (q & 1) ? f1 : f0;
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[mi][q][v] = fmaf(part[mi & 1][q][v], f, acc[mi][q][v]);
        }
      };
      float sx_prev = 0.f;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        Frag nx = cur_f;
        if (mi < 3) {
          nx = frag_at(cur, mi + 1);
          if (spread) {
#pragma unroll
            for (int d = 0; d < (mi < 2 ? 4 : 5); ++d) dma(4 * mi + d, nxt);
          }
        } else if (s + 1 < total_steps) {
          // loads newer than stage s + 1's: stage s + 2's, when this step
          // spread them (and for the other waves, only stores)
          stage_ready(spread || !loader);
          nx = frag_at(nst, 0);
        }
        if (mi < ngrp) mfmas(mi, cur_f);
        if constexpr (F32S) {
          if (mi > 0 && mi - 1 < ngrp) rescale(mi - 1, sx_prev);
          sx_prev = cur_f.sx;
        }
        if (mi == 3 && s + 1 < total_steps && !last) ng = wfrag_at(nst);
        __builtin_amdgcn_sched_barrier(0);
        cur_f = nx;
      }
      if constexpr (F32S) {
        if (3 < ngrp) rescale(3, sx_prev);
      }
      nf = cur_f;
      if (spread) advance();
      if (last) {
        epilogue(ci);
        if (s + 1 < total_steps) ng = wfrag_at(nst);
      }
    };
    if (loader) p_enter(0);
    issue(stg0);
    if (total_steps > 1) issue(stg1);
    stage_ready(total_steps > 1 || !loader);
    nf = frag_at(stg0, 0);
    ng = wfrag_at(stg0);
    int ci = 0, ckb = 0;
    auto adv = [&]() __attribute__((always_inline)) {
      if (++ckb == KB) {
        ckb = 0;
        ++ci;
      }
    };
    for (int s = 0; s < total_steps; s += D8_STAGES) {
      step(std::integral_constant<int, 0>(), s, ci, ckb);
      adv();
      if (s + 1 < total_steps) {
        step(std::integral_constant<int, 1>(), s + 1, ci, ckb);
        adv();
      }
      if (s + 2 < total_steps) {
        step(std::integral_constant<int, 2>(), s + 2, ci, ckb);
        adv();
      }
    }
    __syncthreads();  // the next chunk rewrites desc / rsrc / wsc
  }
}

template <int MODE, bool F32S>
int go_dense8(const SegDesc& s, int topk, float limit, int pow2, hipStream_t st,
              int num_cus) {
  const long grid = 8L * ((num_cus + 7) / 8);
  moe_dense8_kernel<MODE, F32S><<<(unsigned)grid, D8_THREADS, 0, st>>>(s, topk, limit, pow2);
  SLLM_LAUNCHED();
  return 0;
}

}  // namespace

bool dense8_fits(int mode, const SegDesc& s0) {
  return (s0.tile_info ? s0.num_tiles != nullptr : s0.total_rows > 0) &&
         s0.N % (mode == 0 ? 128 : 256) == 0 && s0.K % 128 == 0 &&
         s0.K / 128 <= D8_KBMAX && s0.a && s0.sa && s0.wp && s0.s0 &&
         (mode == 0 ? (s0.hq && s0.hs && s0.s1) : s0.y != nullptr);
}

int launch_dense8(int mode, const SegDesc& s0, int f32s, int topk, float limit,
                  int pow2, hipStream_t st, int num_cus) {
  SLLM_REQUIRE(dense8_fits(mode, s0), "dense fp8 gemm: unsupported segment (N=%d K=%d)",
               s0.N, s0.K);
  SLLM_REQUIRE((s0.tile_info ? (long)s0.max_tiles : (long)s0.total_rows) * s0.N < (1L << 31),
               "dense fp8 gemm: too large");
  if (mode == 0)
    return f32s ? go_dense8<0, true>(s0, topk, limit, pow2, st, num_cus)
                : go_dense8<0, false>(s0, topk, limit, pow2, st, num_cus);
  return f32s ? go_dense8<1, true>(s0, topk, limit, pow2, st, num_cus)
              : go_dense8<1, false>(s0, topk, limit, pow2, st, num_cus);
}

}  // namespace sllm
