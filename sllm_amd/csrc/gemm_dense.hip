// Compute-dense grouped expert GEMM over packed MXFP4 weights, for prefill
// launches whose experts average more than one 128-row tile (a
// DeepSeek-style layer at thousands of tokens, where the matrix cores, the
// LDS and the weight stream all bound the projection).
//
// Same items' arithmetic and outputs as moe_stream_kernel (gemm_stream.hip)
// with the fp4 weight format, over the same packed weights (the outputs
// agree bit for bit); what changes is how operands reach the matrix cores:
// * Wider wave tiles. An item is a 128-row tile x two packed slabs (256 h
//   columns of gate/up, 512 output columns of down); wave w reads packed
//   waves 2 (w % 4) and 2 (w % 4) + 1 of slab 2 np + w / 4 (a contiguous
//   4 KB per K step) and owns 32 h columns (subtiles g, u, g, u) or 64
//   output columns, so each activation fragment read from LDS feeds four
//   MFMAs instead of two.
// * Operands staged in LDS by the gfx950 direct-to-LDS loads
//   (global_load_lds_dwordx4): a K step's weights and its 128 gathered
//   activation rows go to LDS without passing through VGPRs, which leaves
//   the registers to the 128 accumulators of the wider tile. Three LDS
//   stages, loads two steps ahead. The activation rows are XOR-swizzled by
//   row, which keeps the fragment reads free of bank conflicts (the
//   streaming kernel's LDS was in conflict stalls 30% of its cycles at C4).
// * Group mi + 1's LDS reads are issued before group mi's MFMAs; the MFMAs
//   of padding row groups are skipped by a uniform branch around the MFMAs
//   alone (around the reads too, it kept the compiler from issuing them
//   ahead; a second code path for partial tiles does not fit the
//   registers).
//
// Synchronization: a stage is ready when each loader wave has waited for
// its own loads of it (vmcnt, counted per wave: fourteen loads per stage)
// and the waves meet at a barrier without a memory fence -- a fence would
// wait for every load in flight, the prefetched stages included. The
// barrier also orders every wave's reads of the stage before the loads
// that overwrite it. A step makes the next stage ready before its last
// group's MFMAs, so that their issue covers the barrier.
//
// Measured at C4 (cycle counters around each phase of a step, one run,
// all eight waves loading): waves spent ~40% of their time in the MFMA
// phase, ~30% issuing the stage's 64 direct-to-LDS loads right after the
// barrier (the address unit takes them one after another) and ~20% at the
// barrier; issuing the loads between the groups' MFMAs made the step
// slower. Loading by waves 0-3 only (the other wave on each SIMD computes
// meanwhile) took the C4 gate/up launch from 2.16 to 2.07 ms; spreading the
// loaders' loads over their MFMA groups, one load for the weight scales,
// the early barrier and the next step's fragments read under the last
// group's MFMAs, to 1.94 ms (3445 cycles per step against 2048 of MFMA
// issue per SIMD).
#include <type_traits>

#include "launch.h"
#include "lds_dma.h"

namespace sllm {

namespace {

using namespace dma;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int DN_BM = 128;  // rows per tile (the permutation's prefill tiles)
constexpr int DN_WAVES = 8;
constexpr int DN_THREADS = 64 * DN_WAVES;
constexpr int DN_STAGES = 3;
constexpr int DN_ITEMS = 4;                  // items per chunk (LDS row tables)
constexpr int DN_A = DN_BM * 128;            // activations: rows x 128 e4m3
constexpr int DN_B = DN_WAVES * 4 * 1024;    // weights: 4 fp4 subtiles per wave
constexpr int DN_SW = DN_WAVES * 256;        // e8m0 weight scales per wave
constexpr int DN_SX = DN_BM * 4;             // activation scales (fp32)
constexpr int DN_STAGE = DN_A + DN_B + DN_SW + DN_SX;
constexpr int DN_BLK = 16384;                // packed fp4 block (slab, K step)
constexpr int DN_LOADS = 14;                 // direct-to-LDS loads per loader wave per stage

template <int MODE>
__global__ __launch_bounds__(DN_THREADS, 1) void moe_dense_kernel(
    SegDesc S, int topk, float limit, int pow2) {
  // three stages as three arrays: the compiler then sees that a step's LDS
  // reads (one stage) do not alias the loads in flight (the other two) and
  // adds no wait of its own for them
  __shared__ __attribute__((aligned(16))) uint8_t stg0[DN_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stg1[DN_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stg2[DN_STAGE];
  __shared__ int4 desc[DN_ITEMS];
  __shared__ int rsrc[DN_ITEMS][DN_BM];
  __shared__ float rwl[DN_ITEMS][DN_BM];  // row weights (1 without row_w)
  __shared__ float red[DN_BM][DN_WAVES];  // gate/up epilogue: row amax per wave

  constexpr int NTW = MODE == 0 ? 256 : 512;  // columns per item
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4, lc = lane & 15;
  const int K = S.K, KB = K / 128, N = S.N;
  const int ntn = N / NTW;          // items per row tile
  const int nto = N / (NTW / 2);    // packed slabs across N
  const int ow0 = 2 * (wave & 3);   // first packed wave of this wave's pair

  const int total = *S.num_tiles * ntn;
  const int nx = gridDim.x / 8;
  const int xcd = blockIdx.x % 8, jx = blockIdx.x / 8;
  const int xbeg = (int)((long)total * xcd / 8);
  const int xend = (int)((long)total * (xcd + 1) / 8);
  const int nall = xend - xbeg > jx ? (xend - xbeg - jx + nx - 1) / nx : 0;

  for (int cbase = 0; cbase < nall; cbase += DN_ITEMS) {
    const int nitems = min(DN_ITEMS, nall - cbase);
    if (tid < nitems) {
      const int it = xbeg + jx + (cbase + tid) * nx;
      const int rt = it / ntn, np = it % ntn;
      const int4 d = *(const int4*)(S.tile_info + 4 * rt);
      desc[tid] = make_int4(np, d.x, d.y, min(DN_BM, d.z));
    }
    __syncthreads();
    for (int q = tid; q < nitems * DN_BM; q += DN_THREADS) {
      const int i = q / DN_BM, r = q % DN_BM;
      const int4 d = desc[i];
      const int p = d.z + (r < d.w ? r : 0);  // rows past the tile read row 0
      rsrc[i][r] = S.gather ? S.sorted_idx[p] / topk : p;
      rwl[i][r] = S.row_w ? S.row_w[S.row_w_by_idx ? S.sorted_idx[p] : p] : 1.f;
    }
    __syncthreads();
    const int total_steps = nitems * KB;

    // ---- prefetch cursor: per-lane sources of the direct-to-LDS loads ----
    // Waves 0-3 load every stage (waves 4-7 only compute, so that on each
    // SIMD one wave's MFMAs run while the other issues loads; issued by all
    // eight right after the barrier, the loads held every wave at the
    // address unit). Loader L: activation slots 256 L + 64 q + lane (q < 4)
    // of the stage's 1024 16-byte chunks (slot g holds chunk
    // (g % 8) ^ (row % 8) of row g / 8); the weights and weight scales of
    // compute waves 2 L and 2 L + 1; the activation scales of rows 32 L +
    // lane (lane < 32).
    const bool loader = wave < 4;
    int pi = 0, pkb = 0;
    uint32_t poff[4], psx = 0;  // byte offsets from S.a / S.sa
    const uint8_t* pbw[2] = {nullptr, nullptr};   // weight block of wave 2 L + c
    const uint8_t* psw = nullptr;  // scales of both (512 contiguous bytes)
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
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int cw = 2 * wave + c;  // the compute wave served
        const size_t blk = ((size_t)e * nto + 2 * np + (cw >> 2)) * KB;
        pbw[c] = S.wp + blk * DN_BLK + 2 * (cw & 3) * 2048;
        if (c == 0) psw = (const uint8_t*)S.s0 + blk * 1024 + 2 * (cw & 3) * 128;
      }
    };
    // load j (0 <= j < DN_LOADS, a compile-time constant once unrolled) of
    // the loader's stage: 0-3 activation chunks, 4-7 and 8-11 the four
    // weight subtiles of compute waves 2 L and 2 L + 1, 12 their weight
    // scales (512 contiguous bytes, 16 per lane), 13 the activation scales
    auto dma = [&](int j, uint8_t* base) __attribute__((always_inline)) {
      if (j < 4) {
        to_lds(S.a + poff[j] + pkb * 128, base + wave * 4096 + j * 1024, 16);
      } else if (j < 12) {
        const int c = (j - 4) / 4, q = (j - 4) % 4, cw = 2 * wave + c;
        to_lds(pbw[c] + (size_t)pkb * DN_BLK + lane * 16 + q * 1024,
               base + DN_A + cw * 4096 + q * 1024, 16);
      } else if (lane < 32) {
        if (j == 12)
          to_lds(psw + (size_t)pkb * 1024 + lane * 16,
                 base + DN_A + DN_B + 2 * wave * 256, 16);
        else
          to_lds((const uint8_t*)S.sa + psx + pkb * 4,
                 base + DN_A + DN_B + DN_SW + wave * 128, 4);
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
      for (int j = 0; j < DN_LOADS; ++j) dma(j, base);
      advance();
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[mi][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // ---- epilogues --------------------------------------------------------
    // acc[mi][j][v]: token mi * 16 + lc of the tile, output column 4 lg + v
    // of subtile j (gate/up: j = 0, 2 gate and 1, 3 up of packed waves ow0,
    // ow0 + 1; down: columns 16 j + 4 lg + v of the wave's 64).
    auto epilogue = [&](int i) __attribute__((always_inline)) {
      const int4 d = desc[i];
      const int np = d.x, rb = d.z, rows = d.w;
      const int ngrp = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
      const int slab = 2 * np + (wave >> 2);  // packed slab of this wave
      if constexpr (MODE == 0) {
        // h = silu(g) * u * route weight; per-row amax over the four waves
        // of the packed slab (one 128-column quantization block); e4m3
        // with the row's scale
#pragma unroll
        for (int mi = 0; mi < 8; ++mi) {
          if (mi < ngrp) {
            const int t = mi * 16 + lc;
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
            if (lg == 0) red[t][wave] = amax;
          }
        }
        bar_lds();
        const int w0 = wave & 4;  // first wave of this packed slab
#pragma unroll
        for (int mi = 0; mi < 8; ++mi) {
          if (mi < ngrp) {
            const int t = mi * 16 + lc;
            const float amax = fmaxf(fmaxf(red[t][w0], red[t][w0 + 1]),
                                     fmaxf(red[t][w0 + 2], red[t][w0 + 3]));
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
              uint8_t* hrow = S.hq + (size_t)(rb + t) * N + slab * 128;
#pragma unroll
              for (int pr = 0; pr < 2; ++pr) {
                float y[4];
#pragma unroll
                for (int v = 0; v < 4; ++v)
                  y[v] = fminf(fmaxf(acc[mi][2 * pr][v] * inv, -448.f), 448.f);
                *(uint32_t*)(hrow + (ow0 + pr) * 16 + lg * 4) =
                    f32x4_to_e4m3(y[0], y[1], y[2], y[3]);
              }
              if ((wave & 3) == 0 && lg == 0)
                S.hs[(size_t)(rb + t) * (N / 128) + slab] = sc;
            }
          }
        }
      } else {
#pragma unroll
        for (int mi = 0; mi < 8; ++mi) {
          if (mi < ngrp) {
            const int t = mi * 16 + lc;
            if (t < rows) {
              const float rw = rwl[i][t];
              uint16_t* yrow = S.y + (size_t)(rb + t) * N + slab * 256 + ow0 * 32;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const uint32_t lo = pk_bf16(acc[mi][j][0] * rw, acc[mi][j][1] * rw);
                const uint32_t hi = pk_bf16(acc[mi][j][2] * rw, acc[mi][j][3] * rw);
                *(uint2*)(yrow + j * 16 + lg * 4) = make_uint2(lo, hi);
              }
            }
          }
        }
      }
#pragma unroll
      for (int mi = 0; mi < 8; ++mi)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[mi][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };

    // ---- pipeline -----------------------------------------------------------
    // group mi of a step: its activation fragment (with an fp4 A operand
    // the fp8 B operand's two 16-byte halves are K bytes [16 lg, +16) and
    // [64 + 16 lg, +16) of the step, the streaming kernel's fragment for
    // this format) and the row's activation scale
    struct Frag {
      v8i x;
      int sx;
    };
    // a step's weight fragments (the wave's four subtiles) and scales
    // (four named vectors: held in an array, the fragments passed between
    // steps went through the stack)
    struct WFrag {
      u32x4 w0, w1, w2, w3;
      uint32_t sw;
    };
    auto wfrag_at = [&](const uint8_t* stage) __attribute__((always_inline)) {
      const uint8_t* B = stage + DN_A + wave * 4096 + lane * 16;
      const uint8_t* SW = stage + DN_A + DN_B + wave * 256;
      WFrag g;
      g.w0 = *(const u32x4*)(B);
      g.w1 = *(const u32x4*)(B + 1024);
      g.w2 = *(const u32x4*)(B + 2048);
      g.w3 = *(const u32x4*)(B + 3072);
      g.sw = (uint32_t)*(const uint16_t*)(SW + lane * 2) |
             ((uint32_t)*(const uint16_t*)(SW + 128 + lane * 2) << 16);
      return g;
    };
    auto frag_at = [&](const uint8_t* stage, int mi) __attribute__((always_inline)) {
      const int r = mi * 16 + lc;
      const u32x4 x0 = *(const u32x4*)(stage + a_off(r, lg));
      const u32x4 x1 = *(const u32x4*)(stage + a_off(r, 4 + lg));
      const float* SX = (const float*)(stage + DN_A + DN_B + DN_SW);
      Frag f;
      f.x = (v8i){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                  (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
      f.sx = (int)e8m0_of(SX[r]);
      return f;
    };
    // A stage is ready once every loader has waited for its own loads of
    // the stage (vmcnt; the loads of the stage after it may stay in flight:
    // `newer`) and the waves meet at a barrier; each wave's LDS reads are
    // complete by then, so the barrier also ends the reads of the stage
    // that the loads issued after it overwrite.
    auto stage_ready = [&](bool newer) __attribute__((always_inline)) {
      if (newer) wait_vm<DN_LOADS>();
      else wait_vm<0>();
      bar_lds();
    };

    // step s on stage J = s % 3 (J a compile-time constant), K step ckb of
    // item ci, entered with group 0's fragment of the stage; the loaders
    // spread stage s + 2's loads over groups 0-6 (in one burst after the
    // barrier, they held the loader waves at the address unit while the
    // others waited at the next barrier), on an item's last step too
    // (issued after its epilogue, they kept the next item's second step
    // waiting: C4 gate/up 1.98 -> 1.96 ms, down 1.24 -> 1.23 ms). Stage s + 1 is made ready before
    // group 7's MFMAs, whose issue then covers the barrier and the next
    // step's first fragment reads; returns that fragment. The cursors are
    // passed by value: kept in memory, the barrier's memory clobber would
    // make every step reload them.
    Frag nf;    // the next step's first activation fragment
    WFrag ng;   // and its weight fragments
    auto step = [&](auto J, int s, int ci, int ckb) __attribute__((always_inline)) {
      constexpr int j = decltype(J)::value;
      uint8_t* const cur = j == 0 ? stg0 : (j == 1 ? stg1 : stg2);
      uint8_t* const nst = j == 0 ? stg1 : (j == 1 ? stg2 : stg0);
      uint8_t* const nxt = j == 0 ? stg2 : (j == 1 ? stg0 : stg1);
      const bool last = ckb + 1 == KB;
      const bool spread = loader && s + 2 < total_steps;
      Frag cur_f = nf;
      const WFrag g = ng;
      auto mfmas = [&](int mi, const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 w = q == 0 ? g.w0 : (q == 1 ? g.w1 : (q == 2 ? g.w2 : g.w3));
          const v8i wv = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
          acc[mi][q] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              wv, f.x, acc[mi][q], 4, 0, 0, (int)((g.sw >> (8 * q)) & 0xFF), 0, f.sx);
        }
      };
      // the groups' MFMAs (padding groups skipped; the next group's LDS
      // reads are issued first either way), the scheduling barriers keeping
      // the compiler from hoisting every group's reads at once
      const int ngrp = __builtin_amdgcn_readfirstlane((desc[ci].w + 15) >> 4);
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        Frag nx = cur_f;
        if (mi < 7) {
          nx = frag_at(cur, mi + 1);
          if (spread) {
            dma(2 * mi, nxt);
            dma(2 * mi + 1, nxt);
          }
        } else if (s + 1 < total_steps) {
          // loads newer than stage s + 1's: stage s + 2's, when this step
          // spread them (and for the other waves, only stores)
          stage_ready(spread || !loader);
          nx = frag_at(nst, 0);
        }
        if (mi < ngrp) mfmas(mi, cur_f);
        // the next step's weight fragments, read once group 7's MFMAs (the
        // last readers of this step's) are issued
        if (mi == 7 && s + 1 < total_steps && !last) ng = wfrag_at(nst);
        __builtin_amdgcn_sched_barrier(0);
        cur_f = nx;
      }
      nf = cur_f;
      if (spread) advance();
      if (last) {
        epilogue(ci);
        // (read after the epilogue: kept across it, the fragments would not
        // fit the registers)
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
    for (int s = 0; s < total_steps; s += DN_STAGES) {
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
    __syncthreads();  // the next chunk rewrites desc / rsrc
  }
}

template <int MODE>
int go_dense(const SegDesc& s, int topk, float limit, int pow2, hipStream_t st,
             int num_cus) {
  const long grid = 8L * ((num_cus + 7) / 8);
  moe_dense_kernel<MODE><<<(unsigned)grid, DN_THREADS, 0, st>>>(s, topk, limit, pow2);
  SLLM_LAUNCHED();
  return 0;
}

}  // namespace

bool dense_fits(int bf, int mode, const SegDesc& s0, const SegDesc* s1) {
  return bf == 2 && !s1 && s0.wreuse && s0.tile_info && s0.num_tiles &&
         s0.N % (mode == 0 ? 256 : 512) == 0 && s0.K % 128 == 0 &&
         (mode == 0 ? (s0.hq && s0.hs) : s0.y != nullptr);
}

int launch_dense(int mode, const SegDesc& s0, int topk, float limit, int pow2,
                 hipStream_t st, int num_cus) {
  SLLM_REQUIRE(dense_fits(2, mode, s0, nullptr) && s0.a && s0.sa && s0.wp && s0.s0,
               "dense gemm: unsupported segment (N=%d K=%d)", s0.N, s0.K);
  SLLM_REQUIRE((long)s0.max_tiles * s0.N < (1L << 31) && s0.K <= 65536,
               "dense gemm: too large");
  return mode == 0 ? go_dense<0>(s0, topk, limit, pow2, st, num_cus)
                   : go_dense<1>(s0, topk, limit, pow2, st, num_cus);
}

}  // namespace sllm
