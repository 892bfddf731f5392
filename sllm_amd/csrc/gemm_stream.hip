// Persistent, weight-streaming grouped expert GEMMs (prefill) and the packed
// weight layouts they read.
//
// Same arithmetic and epilogues as gemm_grouped.hip (see there for the
// reference semantics); this file changes how the expert weights move and
// how the work is spread over the chip:
//
// * Packed weights. A one-time repack (sllm_moe_pack_weights) stores each
//   expert's weights in MFMA operand order: for every (expert, column slab,
//   128-wide K step) one contiguous block holds, wave by wave and subtile by
//   subtile, exactly the bytes each lane feeds the MFMA, so every wave load
//   instruction reads 1 KB of consecutive HBM and a workgroup streams one
//   contiguous 32 KB (fp8) / 16 KB (fp4) block per K step.
// * Persistent workgroups of eight waves (two per SIMD, so that one wave's
//   LDS, dependency and barrier stalls are covered by the other's MFMA and
//   VALU work), one workgroup per CU. Each walks the flat sequence of
//   (item, K step) of its items, an item being a 128-row tile x column slab
//   of the routed segment or of the shared expert's; operands of step s+3
//   are in flight while step s computes, across item boundaries.
// * XCD-aware item order. Workgroups are dealt to the eight XCDs round-robin
//   (blockIdx % 8). Launches that stream their weights deal the items to
//   the XCDs in chunks of one row tile's items (chunk c to XCD c % 8), so
//   the column slabs of one row tile run at the same time on one XCD and
//   gather the same activation rows through that XCD's L2, and every XCD
//   gets the same mix of routed and shared-expert items. Launches whose
//   weights go through L2 (an expert's tiles share them) give each XCD a
//   contiguous range instead, so that an expert's tiles meet in one L2.
//   Each XCD's workgroups take its items round-robin.
// * Item descriptors and gathered row indices of a workgroup's items are
//   loaded into LDS once at the start.
#include <algorithm>
#include <type_traits>

#include "launch.h"
#include "permute_fused.h"
#include "route_token.h"

namespace sllm {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int ST_BM = 128;
constexpr int ST_LDS = 144;          // A row stride in LDS (128 + 16 pad)
constexpr int ST_MAX_ITEMS = 32;     // work items per workgroup
constexpr int ST_WAVES = 8;          // waves per workgroup
constexpr int ST_THREADS = 64 * ST_WAVES;
// Register sets per operand of the decode kernel's weight stream (prefetch
// distance one less): MXFP4 steps carry 16 KB of weights, FP8 steps 32 KB.
constexpr int DEC_SETS_F4 = 4;
constexpr int DEC_SETS_F8 = 4;
static_assert(ST_THREADS == 4 * ST_BM, "four lanes per activation-scale row");

// ---------------------------------------------------------------------------
// packed layouts
// ---------------------------------------------------------------------------
// up   (MODE 0): W1, W3 (E, N, K), N = intermediate, K = hidden; slab = 128
//       h columns; wave w owns h columns 128 nt + 16 w + (l % 16): subtile 0
//       holds those rows of W1 (gate), subtile 1 the same rows of W3 (up).
// down (MODE 1): W2 (E, N, K), N = hidden, K = intermediate; slab = 256
//       columns; subtile s of wave w = rows 256 nt + 32 w + 16 s + (l % 16).
// fp8: block (e, nt, kb) = 32 KB at ((e NT + nt) KB + kb) * 32768, inside
//       [w 8][s 2][h 2][lane 64][16 B]: the lane's 32 bytes are K
//       [128 kb + 32 (l / 16), +32), half h = bytes [16 h, 16 h + 16).
// fp4: block = 16 KB, [w 8][s 2][lane 64][16 B]: K [128 kb + 32 (l / 16),
//       +32) = packed bytes [64 kb + 16 (l / 16), +16); e8m0 scales packed as
//       1 KB blocks [w 8][lane 64][s 2], byte s = scale of (row of subtile s,
//       K block 4 kb + l / 16).
__device__ __forceinline__ int slab_row(int up, int nt, int w, int s, int l) {
  return up ? nt * 128 + w * 16 + (l & 15)
            : nt * 256 + w * 32 + s * 16 + (l & 15);
}

__global__ void pack_fp8_kernel(const uint8_t* __restrict__ w0,
                                const uint8_t* __restrict__ w1,
                                uint8_t* __restrict__ out, int E, int N, int K,
                                int up) {
  const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int NT = up ? N / 128 : N / 256, KB = K / 128;
  const long nchunks = (long)E * NT * KB * 2048;
  if (c >= nchunks) return;
  const int l = c & 63, h = (c >> 6) & 1, s = (c >> 7) & 1, w = (c >> 8) & 7;
  const long blk = c >> 11;
  const int kb = (int)(blk % KB);
  const long t = blk / KB;
  const int nt = (int)(t % NT), e = (int)(t / NT);
  const int row = slab_row(up, nt, w, s, l);
  const uint8_t* src = (up && s == 1) ? w1 : w0;
  const size_t col = (size_t)kb * 128 + (l >> 4) * 32 + h * 16;
  *(uint4*)(out + c * 16) = *(const uint4*)(src + ((size_t)e * N + row) * K + col);
}

__global__ void pack_fp4_kernel(const uint8_t* __restrict__ w0,
                                const uint8_t* __restrict__ w1,
                                const uint8_t* __restrict__ s0,
                                const uint8_t* __restrict__ s1,
                                uint8_t* __restrict__ out,
                                uint16_t* __restrict__ out_s, int E, int N,
                                int K, int up) {
  const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int NT = up ? N / 128 : N / 256, KB = K / 128;
  const long nchunks = (long)E * NT * KB * 1024;
  if (c >= nchunks) return;
  const int l = c & 63, s = (c >> 6) & 1, w = (c >> 7) & 7;
  const long blk = c >> 10;
  const int kb = (int)(blk % KB);
  const long t = blk / KB;
  const int nt = (int)(t % NT), e = (int)(t / NT);
  const int row = slab_row(up, nt, w, s, l);
  const uint8_t* src = (up && s == 1) ? w1 : w0;
  const size_t col = (size_t)kb * 64 + (l >> 4) * 16;
  *(uint4*)(out + c * 16) =
      *(const uint4*)(src + ((size_t)e * N + row) * (K / 2) + col);
  if (s == 0) {  // one thread per (block, w, lane) writes the two scale bytes
    uint32_t v = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int rq = slab_row(up, nt, w, q, l);
      const uint8_t* sp = (up && q == 1) ? s1 : s0;
      v |= (uint32_t)sp[((size_t)e * N + rq) * (K / 32) + kb * 4 + (l >> 4)]
           << (8 * q);
    }
    out_s[blk * 512 + w * 64 + l] = (uint16_t)v;
  }
}

// ---------------------------------------------------------------------------
// streaming kernel
// ---------------------------------------------------------------------------


// Weight operands of one K step plus their scales (prefetched together so
// that nothing loaded for the current step is issued after the prefetches:
// vmcnt counts loads and stores in order on gfx9, so a late load would make
// the wait for it drain every prefetch behind it).
template <int BF>
struct BSet {
  v8i v[2];
  uint32_t sc;   // fp4: packed e8m0 scale bytes of the 2 subtiles
  float sb0;     // fp8: W1 / W2 block scale
  float sb1;     // fp8 gate/up: W3 block scale
};

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Streaming (nontemporal) 16-byte load: expert weights are read once per
// layer and should not evict the gathered activation rows from L2.
// WNT = false: an ordinary load, for launches whose experts span several
// row tiles, so that the tiles of one expert (streamed at the same time on
// one XCD) share the weights through L2.
template <bool WNT>
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  if constexpr (WNT) {
    const v4u t = __builtin_nontemporal_load((const v4u*)p);
    return make_uint4(t.x, t.y, t.z, t.w);
  } else {
    return *(const uint4*)p;
  }
}

// Set (to 1) by a decode streamed launch whose workgroup was dealt more
// than ST_MAX_ITEMS items, which it then leaves undone: the host sizes the
// grid from a bound of the item count, so this marks a host sizing error
// (the prefill kernel takes any item count, in chunks). One word per device
// (zero at load); sllm_moe_stream_status reads and clears it.
__device__ int stream_item_overflow;

template <int MODE>
__device__ __forceinline__ int seg_items(const SegDesc& s) {
  const int ntn = MODE == 0 ? s.N / 128 : s.N / 256;
  const int rt = s.tile_info ? *s.num_tiles : (s.total_rows + ST_BM - 1) / ST_BM;
  return rt * ntn;
}

__device__ __forceinline__ uint32_t e8m0_bits(float pow2) {
  return (__float_as_uint(pow2) >> 23) & 0xFF;
}

// One 16x16x128 MFMA with the weights as operand A and the activations as
// operand B: lane l then holds D[4 (l / 16) + v][l % 16], i.e. four
// consecutive output columns (v) of token l % 16. sw / sx are the e8m0
// scales of the weight row and of the token (ignored for SF_FP8_F32S, whose
// block scales are applied to the unscaled partial by the caller).
template <int BF>
__device__ __forceinline__ f32x4 st_mma(const v8i& w, const v8i& x, f32x4 c,
                                        uint32_t sw, uint32_t sx) {
  if constexpr (BF == SF_FP8_F32S) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, x, z, 0, 0, 0,
                                                            0, 0, 0);
  } else if constexpr (BF == SF_FP8_POW2) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        w, x, c, 0, 0, 0, (int)sw, 0, (int)sx);
  } else {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        w, x, c, 4, 0, 0, (int)sw, 0, (int)sx);
  }
}

template <int BF, int MODE>
struct Stream {
  static constexpr int NTW = MODE == 0 ? 128 : 256;
  static constexpr int BLK = BF == SF_FP4 ? 16384 : 32768;
};

// Scheduling pattern of one prefill step: before each of the eight pairs of
// MFMAs (one 16-row group), one or two of the step's prefetch loads. Spreading the loads keeps the workgroup's
// burst of vector loads after the barrier from backing up the address unit
// while the matrix cores idle.
#define ST_SCHED_GROUP(nv)                                   \
  do {                                                       \
    if ((nv) > 0) __builtin_amdgcn_sched_group_barrier(0x0020, (nv), 0); \
    __builtin_amdgcn_sched_group_barrier(0x0008, 2, 0);      \
  } while (0)

template <int NV>
__device__ __forceinline__ void st_sched_pattern() {
  // NV prefetch loads over eight groups: the first NV - 8 groups take two
  constexpr int e = NV > 8 ? NV - 8 : 0;
  constexpr int one = NV > 8 ? 1 : 0;
  ST_SCHED_GROUP(e > 0 ? 2 : (0 < NV ? 1 : 0));
  ST_SCHED_GROUP(e > 1 ? 2 : (1 < NV || one ? 1 : 0));
  ST_SCHED_GROUP(e > 2 ? 2 : (2 < NV || one ? 1 : 0));
  ST_SCHED_GROUP(e > 3 ? 2 : (3 < NV || one ? 1 : 0));
  ST_SCHED_GROUP(e > 4 ? 2 : (4 < NV || one ? 1 : 0));
  ST_SCHED_GROUP(e > 5 ? 2 : (5 < NV || one ? 1 : 0));
  ST_SCHED_GROUP(e > 6 ? 2 : (6 < NV || one ? 1 : 0));
  ST_SCHED_GROUP(e > 7 ? 2 : (7 < NV || one ? 1 : 0));
}

// item descriptor in LDS: x = seg | nt << 1, y = e, z = row_begin, w = rows
// Activation scales: with every K a multiple of 512 (PERSTEP false), items
// are whole groups of four steps, and the second step of each unrolled
// four-step body loads the scales of the next group -- lane (row tid / 4,
// block tid % 4), one 4-byte load, a wave touching 16 rows -- which the
// first step of the next body stores to LDS. Otherwise (PERSTEP) each step
// loads its own scale, four lanes per row.
template <int BF, int MODE, bool PERSTEP, bool WNT>
__global__ __launch_bounds__(ST_THREADS, 1) void moe_stream_kernel(
    SegDesc S0, SegDesc S1, int nseg, int topk, float limit, int pow2) {
  constexpr int YS = 264;  // bf16 row stride of the down-projection staging
  __shared__ int4 desc[ST_MAX_ITEMS];
  __shared__ int rsrc[ST_MAX_ITEMS][ST_BM];
  __shared__ float rwl[ST_MAX_ITEMS][ST_BM];
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][ST_BM * ST_LDS];
  // activation scales of the tile rows: per four-step group (double
  // buffered by group parity), or per step (PERSTEP)
  __shared__ __attribute__((aligned(16))) float sa_lds[2][ST_BM][PERSTEP ? 1 : 4];
  __shared__ __attribute__((aligned(16))) float red[ST_BM][ST_WAVES];
  __shared__ __attribute__((aligned(16))) uint16_t ystage[MODE == 1 ? ST_BM * YS : 8];

  constexpr int NTW = Stream<BF, MODE>::NTW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, lc = lane & 15;

  // ---- this workgroup's items (XCD-aware round-robin) ----------------------
  const int n0 = seg_items<MODE>(S0);
  const int n1 = nseg > 1 ? seg_items<MODE>(S1) : 0;
  const int total = n0 + n1;
  const int nx = gridDim.x / 8;  // workgroups per XCD (grid is a multiple of 8)
  const int xcd = blockIdx.x % 8, jx = blockIdx.x / 8;
  // Items to XCDs. Weights through L2 (wreuse: an expert's row tiles share
  // its weights): each XCD a contiguous range of the items, so that an
  // expert's tiles meet in one L2. Streamed weights: XCD x takes chunks x,
  // x + 8, ... of CB consecutive items (one routed row tile's column slabs,
  // which share its gathered rows in L2), so that every XCD gets the same
  // mix of items -- with contiguous ranges the last XCD got the shared
  // expert's tiles, whose weights stay in L2, and finished early while the
  // others streamed (C2 gate/up 244-247 -> 218-219 us; C5, where an
  // expert's tiles then spread over the XCDs, 567 -> 580-588 us).
  const bool ranges = S0.wreuse != 0;
  const int CB = max(1, S0.N / NTW);
  const int ncf = total / CB, crem = total % CB;
  const int xbeg = (int)((long)total * xcd / 8);
  const int xend = (int)((long)total * (xcd + 1) / 8);
  const int xcount = ranges ? xend - xbeg
                            : (ncf > xcd ? (ncf - xcd + 7) / 8 : 0) * CB +
                                  (ncf % 8 == xcd ? crem : 0);
  const int nall = xcount > jx ? (xcount - jx + nx - 1) / nx : 0;
  // The items are taken ST_MAX_ITEMS at a time (the LDS holds the row
  // indices and weights of that many): one pipeline per chunk, so that the
  // grid stays at one workgroup per CU whatever the item count.
  for (int cbase = 0; cbase < nall; cbase += ST_MAX_ITEMS) {
  const int nitems = min(ST_MAX_ITEMS, nall - cbase);
  auto item_at = [&](int m) {
    const int q = jx + (cbase + m) * nx;  // the XCD's q-th item
    return ranges ? xbeg + q : (xcd + 8 * (q / CB)) * CB + q % CB;
  };

  // ---- phase 0: descriptors and gathered row indices -> LDS ---------------
  if (tid < nitems) {
    const int it = item_at(tid);
    const int seg = it >= n0;
    const SegDesc& S = seg ? S1 : S0;
    const int li = seg ? it - n0 : it;
    const int ntn = S.N / NTW;
    const int rt = li / ntn, nt = li % ntn;
    int e = 0, rb, rows;
    if (S.tile_info) {
      const int4 d = *(const int4*)(S.tile_info + 4 * rt);
      e = d.x;
      rb = d.y;
      rows = min(ST_BM, d.z);
    } else {
      rb = rt * ST_BM;
      rows = min(ST_BM, S.total_rows - rb);
    }
    desc[tid] = make_int4(seg | (nt << 1), e, rb, rows);
  }
  __syncthreads();
  for (int q = tid; q < nitems * ST_BM; q += ST_THREADS) {
    const int i = q / ST_BM, r = q % ST_BM;
    const int4 d = desc[i];
    const SegDesc& S = (d.x & 1) ? S1 : S0;
    int src = 0;
    float rw = 1.f;
    if (r < d.w) {
      const int p = d.z + r;
      src = S.gather ? S.sorted_idx[p] / topk : p;
      if (S.row_w) rw = S.row_w[S.row_w_by_idx ? S.sorted_idx[p] : p];
    }
    rsrc[i][r] = src;
    rwl[i][r] = rw;
  }
  __syncthreads();

  // ---- per-step helpers ---------------------------------------------------
  auto kb_of = [&](int i) {
    const int4 d = desc[i];
    return ((d.x & 1) ? S1.K : S0.K) / 128;
  };
  int total_steps = 0;
  for (int i = 0; i < nitems; ++i) total_steps += kb_of(i);

  struct ASet {
    uint4 v[2];
    float s;  // PERSTEP: the row's scale of this step
  };

  // ---- prefetch cursor ------------------------------------------------------
  // Addresses of the prefetch cursor's item are kept in registers and
  // rebuilt from LDS only when the cursor enters a new item, so a step's
  // loads issue without a chain of dependent LDS reads.
  // Thread tid gathers 16-byte chunk (tid & 7) of tile rows 64 q + tid / 8:
  // each load instruction of a wave reads eight whole 128-byte row segments.
  // Rows past the tile read the valid row 0 of rsrc; they are zeroed when
  // the registers are stored to LDS, after the wait (a load under a branch,
  // which is what the compiler makes of a select applied right after the
  // load, leaves it no guaranteed count of younger loads and forces a wait
  // that drains the pipeline).
  const int a_chunk = tid & 7, a_row0 = tid >> 3;
  int pi = 0, pkb = 0, pKB = 1;
  const uint8_t *pa0 = nullptr, *pa1 = nullptr, *pb = nullptr;
  const float *psa = nullptr, *ps0 = nullptr, *ps1 = nullptr;
  float sgrp = 0.f;  // !PERSTEP: scale of (row tid / 4, block tid % 4) of a group
  const uint16_t* ps4 = nullptr;
  auto p_enter = [&](int i) {
    const int4 d = desc[i];
    const int seg = d.x & 1, nt = d.x >> 1;
    const SegDesc& S = seg ? S1 : S0;
    const int K = S.K, KB = K / 128, N = S.N, NT = N / NTW;
    pKB = KB;
    pa0 = S.a + (size_t)rsrc[i][a_row0] * K + a_chunk * 16;
    pa1 = S.a + (size_t)rsrc[i][64 + a_row0] * K + a_chunk * 16;
    // four lanes share each activation-scale row (a wave's scale load
    // touches 16 rows)
    psa = S.sa + (size_t)rsrc[i][tid >> 2] * KB;
    const size_t blk0 = ((size_t)d.y * NT + nt) * KB;
    if constexpr (BF == SF_FP4) {
      pb = S.wp + blk0 * Stream<BF, MODE>::BLK + (wave * 2) * 1024 + lane * 16;
      ps4 = (const uint16_t*)S.s0 + blk0 * 512 + wave * 64 + lane;
    } else {
      pb = S.wp + blk0 * Stream<BF, MODE>::BLK + (wave * 4) * 1024 + lane * 16;
      // the block scales are wave-uniform: read through the scalar cache
      // (constant address space), off the vector memory path
      const int ue = __builtin_amdgcn_readfirstlane(d.y);
      const int unt = __builtin_amdgcn_readfirstlane(nt);
      if constexpr (MODE == 0) {
        const size_t ub0 = ((size_t)ue * NT + unt) * KB;  // NT = N / 128
        ps0 = (const float*)S.s0 + ub0;
        ps1 = (const float*)S.s1 + ub0;
      } else {
        const int nblk = unt * 2 + __builtin_amdgcn_readfirstlane(wave) / 4;
        ps0 = ps1 = (const float*)S.s0 + ((size_t)ue * (N / 128) + nblk) * KB;
      }
    }
  };
  auto p_advance = [&]() {  // saturates at the last step of the last item
    if (pkb + 1 < pKB) {
      ++pkb;
    } else if (pi + 1 < nitems) {
      ++pi;
      pkb = 0;
      p_enter(pi);
    }
  };
  // the group of four steps starting at the prefetch cursor (pkb % 4 == 0)
  auto p_group_scales = [&]() { sgrp = psa[pkb + (tid & 3)]; };
  auto fetch_a = [&](ASet& af) {
    af.v[0] = *(const uint4*)(pa0 + pkb * 128);
    af.v[1] = *(const uint4*)(pa1 + pkb * 128);
    if constexpr (PERSTEP) af.s = psa[pkb];
  };
  auto load_b = [&](BSet<BF>& b) {
    const uint8_t* base = pb + (size_t)pkb * Stream<BF, MODE>::BLK;
    if constexpr (BF == SF_FP4) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint4 v = ld_stream<WNT>(base + s * 1024);
        b.v[s] = (v8i){(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
      }
      b.sc = __builtin_nontemporal_load(ps4 + (size_t)pkb * 512);
      b.sb0 = b.sb1 = 0.f;
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint4 lo4 = ld_stream<WNT>(base + (2 * s) * 1024);
        const uint4 hi4 = ld_stream<WNT>(base + (2 * s + 1) * 1024);
        b.v[s] = (v8i){(int)lo4.x, (int)lo4.y, (int)lo4.z, (int)lo4.w,
                       (int)hi4.x, (int)hi4.y, (int)hi4.z, (int)hi4.w};
      }
      b.sc = 0;
      typedef const __attribute__((address_space(4))) float* cfp;
      b.sb0 = ((cfp)ps0)[pkb];
      b.sb1 = MODE == 0 ? ((cfp)ps1)[pkb] : b.sb0;
    }
  };

  f32x4 acc[8][2];
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
#pragma unroll
    for (int s = 0; s < 2; ++s) acc[mi][s] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // ---- compute cursor -------------------------------------------------------
  int ci = 0, ckb = 0, cKB = 1, crows = 0;
  auto c_enter = [&](int i) {
    const int4 d = desc[i];
    cKB = ((d.x & 1) ? S1.K : S0.K) / 128;
    crows = d.w;
  };

  // ---- epilogues ------------------------------------------------------------
  // acc[mi][s][v] holds token mi * 16 + lc (tile row) and output column
  // 4 lg + v of the wave's subtile s.
  auto epilogue = [&](int i, int ebuf) {
    const int4 d = desc[i];
    const int seg = d.x & 1, nt = d.x >> 1;
    const SegDesc& S = seg ? S1 : S0;
    const int rows = d.w, rb = d.z;
    const int nmi = (rows + 15) >> 4;
    if constexpr (MODE == 0) {
      // h = silu(g) * u * route weight over the wave's 16 columns, row amax
      // across lane groups and then across the eight waves, requantised per
      // row (one 128-column block) to e4m3.
      const int ntn = S.N / 128;
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        if (mi < nmi) {
          const int t = mi * 16 + lc;
          const float rw = rwl[i][t];
          float amax = 0.f;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float g = acc[mi][0][v], u = acc[mi][1][v];
            if (limit > 0.f) {
              u = fminf(fmaxf(u, -limit), limit);
              g = fminf(g, limit);
            }
            const float h = silu_fast(g) * u * rw;
            acc[mi][0][v] = h;
            amax = fmaxf(amax, fabsf(h));
          }
          amax = rows4_max(amax);
          if (lg == 0) red[t][wave] = amax;
        }
      }
      __syncthreads();
      uint8_t* h_lds = a_lds[ebuf];
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        if (mi < nmi) {
          const int t = mi * 16 + lc;
          const float4 r0 = *(const float4*)&red[t][0];
          const float4 r1 = *(const float4*)&red[t][4];
          const float amax = fmaxf(fmaxf(fmaxf(r0.x, r0.y), fmaxf(r0.z, r0.w)),
                                   fmaxf(fmaxf(r1.x, r1.y), fmaxf(r1.z, r1.w)));
          float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
          float inv;
          if (pow2) {  // power-of-two scale: its reciprocal is exact
            const uint32_t bits = __float_as_uint(sc);
            const int ex = (int)((bits >> 23) & 0xFF) - 127 +
                           ((bits & 0x7FFFFF) ? 1 : 0);
            sc = __uint_as_float((uint32_t)(ex + 127) << 23);
            inv = __uint_as_float((uint32_t)(127 - ex) << 23);
          } else {
            inv = __builtin_amdgcn_rcpf(sc);  // within 1 ulp of 1 / sc
          }
          float y[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            y[v] = fminf(fmaxf(acc[mi][0][v] * inv, -448.f), 448.f);
          *(uint32_t*)(h_lds + t * ST_LDS + wave * 16 + lg * 4) =
              f32x4_to_e4m3(y[0], y[1], y[2], y[3]);
          if (wave == 0 && lg == 0 && t < rows)
            S.hs[(size_t)(rb + t) * ntn + nt] = sc;
        }
      }
      __syncthreads();
      // streaming stores: h is read back only by the next kernel
      for (int c = tid; c < rows * 8; c += ST_THREADS) {
        const int r = c >> 3, c16 = c & 7;
        __builtin_nontemporal_store(*(const v4u*)(h_lds + r * ST_LDS + c16 * 16),
                                    (v4u*)(S.hq + (size_t)(rb + r) * S.N + nt * 128 + c16 * 16));
      }
      __syncthreads();  // h_lds is the next step's A buffer
    } else {
      // y = acc * row weight as bf16, staged in LDS (four consecutive
      // columns per lane = one 8-byte write), then 16-byte row stores
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        if (mi < nmi) {
          const int t = mi * 16 + lc;
          const float w = rwl[i][t];
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const uint32_t lo = pk_bf16(acc[mi][s][0] * w, acc[mi][s][1] * w);
            const uint32_t hi = pk_bf16(acc[mi][s][2] * w, acc[mi][s][3] * w);
            *(uint2*)(ystage + t * YS + wave * 32 + s * 16 + lg * 4) =
                make_uint2(lo, hi);
          }
        }
      }
      __syncthreads();
      for (int c = tid; c < rows * 32; c += ST_THREADS) {
        const int r = c >> 5, c8 = c & 31;
        *(uint4*)(S.y + (size_t)(rb + r) * S.N + nt * 256 + c8 * 8) =
            *(const uint4*)(ystage + r * YS + c8 * 8);
      }
      __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
      for (int s = 0; s < 2; ++s) acc[mi][s] = (f32x4){0.f, 0.f, 0.f, 0.f};
  };


  // ---- one pipeline step ----------------------------------------------------
  // j: the step's position in the unrolled four-step body
  auto step = [&](int st, int j, ASet& acur, ASet& aload, BSet<BF>& bcur,
                  BSet<BF>& bload) {
    const int buf = st & 1;
    {  // A(st) registers -> LDS, rows past the tile zeroed
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int r = q * 64 + a_row0;
        const uint32_t m = r < crows ? ~0u : 0u;
        const uint4 v = acur.v[q];
        *(uint4*)(a_lds[buf] + r * ST_LDS + a_chunk * 16) =
            make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
      }
      const uint32_t ms = (tid >> 2) < crows ? ~0u : 0u;
      if constexpr (PERSTEP) {
        if ((tid & 3) == 0)
          sa_lds[buf][tid >> 2][0] = __uint_as_float(__float_as_uint(acur.s) & ms);
      } else if (j == 0) {  // this group's scales, loaded three steps ago
        sa_lds[(st >> 2) & 1][tid >> 2][tid & 3] =
            __uint_as_float(__float_as_uint(sgrp) & ms);
      }
    }
    __syncthreads();
    // both operands are prefetched three steps ahead; the activations of a
    // step are consumed before its weights, so they are issued first. The
    // batch is issued in the same order in every step and in the prologue,
    // so the compiler's count of younger loads at each wait is the same on
    // every path into it; the cursor advances before the loads (its item
    // change is a branch), keeping the loads, LDS reads and MFMAs in one
    // scheduling region.
    p_advance();
    if (!PERSTEP && j == 1) p_group_scales();
    fetch_a(aload);
    load_b(bload);
    // compute step st over all eight 16-row groups: rows past the tile are
    // zero in LDS, and a branch-free step lets the compiler issue the LDS
    // reads of the next groups ahead of the MFMAs of the current one.
    const uint8_t* lds = a_lds[buf];
    // 16-row groups holding tile rows (wave-uniform): the e8m0-scaled
    // MFMAs of the padding groups past them are skipped (C4: gate/up 2.37 ->
    // 2.32 ms, down 1.32 -> 1.24). The fp32-scale path keeps its
    // branch-free group loop: skipping there made C2's gate/up 10% slower
    // and C5's (whose cold experts leave half-empty second tiles) 25%.
    const int ngrp = __builtin_amdgcn_readfirstlane((crows + 15) >> 4);
    auto sx_of = [&](int row) -> float {  // activation scale of a tile row
      if constexpr (PERSTEP) return sa_lds[buf][row][0];
      else return sa_lds[(st >> 2) & 1][row][st & 3];
    };
    auto a_frag = [&](int mi) {
      const uint8_t* row = lds + (mi * 16 + lc) * ST_LDS;
      const uint8_t* p0 = BF == SF_FP4 ? row + lg * 16 : row + lg * 32;
      const uint8_t* p1 = BF == SF_FP4 ? row + 64 + lg * 16 : row + lg * 32 + 16;
      const uint4 x0 = *(const uint4*)p0, x1 = *(const uint4*)p1;
      return (v8i){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                   (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    };
    if constexpr (BF == SF_FP8_F32S) {
      // fp32 block scales: each MFMA yields the unscaled partial of one
      // 128-wide K block, added as acc += partial * (s_x[token] * s_w); the
      // lane's four values share one token. The MFMAs of row group mi run
      // while the partials of group mi - 1 are rescaled, from a second set
      // of partial registers.
      const float sb0 = bcur.sb0, sb1 = MODE == 0 ? bcur.sb1 : bcur.sb0;
      f32x4 part[2][2];
      auto rescale = [&](int m) {
        const float sx = sx_of(m * 16 + lc);
        const float f0 = sx * sb0, f1 = sx * sb1;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const float f = s == 0 ? f0 : f1;
#pragma unroll
          for (int v = 0; v < 4; ++v)
            acc[m][s][v] = fmaf(part[m & 1][s][v], f, acc[m][s][v]);
        }
      };
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        const v8i x = a_frag(mi);
#pragma unroll
        for (int s = 0; s < 2; ++s)
          part[mi & 1][s] = st_mma<BF>(bcur.v[s], x, part[mi & 1][s], 0, 0);
        if (mi > 0) rescale(mi - 1);
      }
      rescale(7);
    } else {
      uint32_t sbe[2];
      if constexpr (BF == SF_FP4) {
        sbe[0] = bcur.sc & 0xFF;
        sbe[1] = (bcur.sc >> 8) & 0xFF;
      } else {
        sbe[0] = e8m0_bits(bcur.sb0);
        sbe[1] = e8m0_bits(MODE == 0 ? bcur.sb1 : bcur.sb0);
      }
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        if (mi < ngrp) {
          const v8i x = a_frag(mi);
          const uint32_t sxe = e8m0_bits(sx_of(mi * 16 + lc));
#pragma unroll
          for (int s = 0; s < 2; ++s)
            acc[mi][s] = st_mma<BF>(bcur.v[s], x, acc[mi][s], sbe[s], sxe);
        }
      }
    }
    st_sched_pattern<BF == SF_FP4 ? 6 : 7>();
    if (++ckb == cKB) {
      epilogue(ci, buf ^ 1);
      ckb = 0;
      if (ci + 1 < nitems) c_enter(++ci);
    }
  };

  // ---- pipeline -------------------------------------------------------------
  // Four register sets per operand, prefetch distance 3. The loop body runs
  // its four steps unconditionally: a conditional step would make the
  // compiler's wait analysis at the back-edge merge a path whose most recent
  // loads are older, and wait for everything.
  BSet<BF> b0, b1, b2, b3;
  ASet a0, a1, a2, a3;
  p_enter(0);
  if (!PERSTEP) p_group_scales();
  c_enter(0);
  fetch_a(a0);
  load_b(b0);
  p_advance();
  fetch_a(a1);
  load_b(b1);
  p_advance();
  fetch_a(a2);
  load_b(b2);
  int st = 0;
  for (; st + 4 <= total_steps; st += 4) {
    step(st, 0, a0, a3, b0, b3);
    step(st + 1, 1, a1, a0, b1, b0);
    step(st + 2, 2, a2, a1, b2, b1);
    step(st + 3, 3, a3, a2, b3, b2);
  }
  // (only PERSTEP totals leave a remainder: otherwise every item is whole
  // groups of four steps)
  if (st < total_steps) step(st, 0, a0, a3, b0, b3);
  if (st + 1 < total_steps) step(st + 1, 1, a1, a0, b1, b0);
  if (st + 2 < total_steps) step(st + 2, 2, a2, a1, b2, b1);
  __syncthreads();  // the next chunk restages desc / rsrc / rwl
  }  // chunks
}

// ---------------------------------------------------------------------------
// decode variant
// ---------------------------------------------------------------------------
// Same items, packed weights, persistent XCD-aware dealing and prefetch
// pipeline as moe_stream_kernel, for the decode regime (a handful of rows
// per expert): 16- or 32-row tiles, activations kept unquantized. Each lane's
// weight bytes (32 consecutive K of its row) are converted to bf16 in
// registers -- exact for e4m3 and for e2m1 times its e8m0 scale -- and fed to
// four v_mfma_f32_16x16x32_bf16 per subtile and K step, slice m taking K
// [32 g + 8 m, +8) of lane group g for both operands. x is bf16 already;
// the fp32 h of the down projection is split into bf16 hi + lo halves (two
// MFMAs), which keeps ~16 mantissa bits. fp8 block scales multiply the
// step's fp32 partial.
constexpr int SD_LS = 136;  // bf16 row stride of the LDS activation tile

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int v4uv __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_bf16_hi(float a, float b) {
  // fp32 values that are exact in bf16: keep the upper halves
  return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xFFFF0000u);
}

// 8 e4m3 bytes (two dwords) -> 8 bf16
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t d0, uint32_t d1) {
  const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(d0, false);
  const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(d0, true);
  const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(d1, false);
  const f32x2 e = __builtin_amdgcn_cvt_pk_f32_fp8(d1, true);
  const v4uv r = {pack_bf16_hi(a.x, a.y), pack_bf16_hi(b.x, b.y),
                    pack_bf16_hi(c.x, c.y), pack_bf16_hi(e.x, e.y)};
  return __builtin_bit_cast(bf16x8, r);
}

// 8 e2m1 values (one dword, low nibble first) times the e8m0 scale byte sb
// -> 8 bf16, exact: v_cvt_scalef32_pk_bf16_fp4 converts the two nibbles of
// byte j (low nibble first) times 2^(exponent of its f32 scale operand - 127)
// in one instruction. Checked on gfx950 against e2m1 * 2^(sb - 127) in fp32
// for every data byte and scale byte: bit-identical, denormals included, for
// sb 1..254, and NaN for sb 255, as the loader convention has it
// (loaders/fp8.py:145-156). The instruction reads sb 0 as 2^-127, where the
// convention has a zero scale: the data word is zeroed instead (+0 for -0
// products, which leaves every sum unchanged).
__device__ __forceinline__ bf16x8 fp4x8_to_bf16(uint32_t d, uint32_t sb) {
  d = sb ? d : 0u;
  const float s = __uint_as_float(sb << 23);
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 0);
  const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 1);
  const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 2);
  const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 3);
  const v4uv r = {__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                  __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
  return __builtin_bit_cast(bf16x8, r);
}

// BM: rows per tile, 16 or 32 (RB = BM / 16 row blocks; each weight
// fragment feeds one MFMA per row block).
// Device-scope accesses of the fused gate/up finish's chunk sums (buffer
// instructions with the sc1 cache policy): stores write through the XCD's
// L2 to the device's coherence point and loads do not take a line from the
// reading XCD's L2, so the sums cross XCDs without the whole-L2 write-back
// and invalidate of device-scope fences (a fence pair per workgroup made a
// B=32 layer 1.3x slower). `base` must be the same in every lane of the
// wave.
constexpr int CP_SC1 = 16;  // buffer cache policy bit of device scope

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const float* base) {
  const uint64_t a = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(
      (void*)(((uint64_t)hi << 32) | lo), 0, 0x7FFFFFF0, 0x00020000);
}

__device__ __forceinline__ void st_dev4(__amdgpu_buffer_rsrc_t r, long off,
                                        float a, float b, float c, float d) {
  const v4uv v = {__float_as_uint(a), __float_as_uint(b), __float_as_uint(c),
                  __float_as_uint(d)};
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)(off * 4), 0, CP_SC1);
}

__device__ __forceinline__ float4 ld_dev4(__amdgpu_buffer_rsrc_t r, long off) {
  const v4uv v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off * 4), 0, CP_SC1);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y),
                     __uint_as_float(v.z), __uint_as_float(v.w));
}

// Fused finish of a K-split gate/up decode launch (DecFuse, launch.h), run
// by every workgroup after its last item. Its chunk sums were stored at
// device scope; each thread waits for its own stores to complete (vmcnt 0:
// written through to the coherence point) before the barrier, after which
// one thread per item counts the arrival of its chunk. The workgroup that
// brings an item's count to ksplit reads the item's chunk sums at device
// scope and computes h as split_finish_kernel does (chunks added in order,
// then the clamps and SiLU). An item's sums are read only there, so no XCD
// holds an older copy of them from this launch; earlier launches' copies
// are gone with the L2 invalidation at every launch's start.
template <int BM>
__device__ __forceinline__ void dec_fused_finish(
    const SegDesc& S0, const SegDesc& S1, float limit, const DecFuse& F,
    const int4* desc, const int4* kr, int nitems, int* jobs, int& njob) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores done
  if (tid == 0) njob = 0;
  __syncthreads();
  for (int i = tid; i < nitems; i += ST_THREADS) {
    const int4 d = desc[i];
    const int seg = d.x & 1, nt = (d.x >> 1) & 0x7FFF;
    const SegDesc& S = seg ? S1 : S0;
    if (S.ksplit <= 1) continue;  // finished in the item's epilogue
    int* c = F.cnt + (seg ? F.cnt1 : 0) + (long)d.z * (S.N / 128) + nt;
    // A relaxed device-scope count. The ordering it relies on is the
    // ISA's, not the HIP memory model's: every chunk sum went out as a
    // device-scope (sc1) store, written through this XCD's L2 to the
    // coherence point, and each thread waited for its own stores'
    // completion (vmcnt 0) before the barrier above, so they are visible
    // device-wide before any count of this workgroup issues; the finisher
    // learns it finished from the count's return value, and its loads of
    // the sums, issued only after that (in order, no speculation), are
    // device-scope (sc1) loads that miss any stale L2 copy. An acq_rel
    // count (a whole-L2 write-back before it and an L2 invalidate after)
    // gives the same bits and cost B=1 / 2 / 4 layers 2 / 7 / 7.5 us.
    // (a stream-K unit's first item also arrives for its zero slices)
    const int inc = 1 + kr[i].z;
    if (__hip_atomic_fetch_add(c, inc, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT) == S.ksplit - inc)
      jobs[atomicAdd(&njob, 1)] = i;
  }
  __syncthreads();
  const int nj = njob;
  // a wave per finished item: its rows x 128 columns, four columns per lane
  for (int j = wave; j < nj; j += ST_THREADS / 64) {
    const int4 d = desc[__builtin_amdgcn_readfirstlane(jobs[j])];
    const int nt = (d.x >> 1) & 0x7FFF;
    const SegDesc& S = (d.x & 1) ? S1 : S0;
    const __amdgpu_buffer_rsrc_t rp = dev_rsrc(S.pp);
    const int ks = S.ksplit;
    for (int q = lane; q < d.w * 32; q += 64) {
      const int row = q / 32, c4 = q % 32;
      const long o = (long)(d.z + row) * S.N + nt * 128 + c4 * 4;
      float gs[4] = {0.f, 0.f, 0.f, 0.f}, us[4] = {0.f, 0.f, 0.f, 0.f};
      for (int k = 0; k < ks; ++k) {
        const float4 g = ld_dev4(rp, k * S.pstride + o);
        const float4 u = ld_dev4(rp, (ks + k) * S.pstride + o);
        gs[0] += g.x; gs[1] += g.y; gs[2] += g.z; gs[3] += g.w;
        us[0] += u.x; us[1] += u.y; us[2] += u.z; us[3] += u.w;
      }
      float h[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float gv = gs[v], uv = us[v];
        if (limit > 0.f) {
          uv = fminf(fmaxf(uv, -limit), limit);
          gv = fminf(gv, limit);
        }
        h[v] = silu_f32(gv) * uv;
      }
      *(float4*)((float*)S.hq + o) = make_float4(h[0], h[1], h[2], h[3]);
    }
  }
}

// Fused combine of a decode down launch (DecCombine, launch.h), run by
// every workgroup after its last item, with the ordering argument of
// dec_fused_finish: the y slices went out as device-scope (sc1) stores,
// each thread waits for its own (vmcnt 0) before the barrier, and the
// finisher reads the slices with device-scope loads once the count's
// return value says its arrival was the unit's last. A unit (token t,
// 256-column slab) expects one arrival per K slice of each kept slot of t
// and per shared-expert slice. Its sum is launch_combine_split's: a group
// of four waves takes the slices (slot-major, then K slice, then shared)
// w, w + 4, ... in batches of CF_BATCH loads, and the four partial sums
// are added in wave order; the two wave groups take a unit each.
constexpr int DC_BATCH = 8;  // combine_f32_kernel's batch of slice loads

template <int BM>
__device__ __forceinline__ void dec_fused_combine(
    const SegDesc& S0, const SegDesc& S1, const DecCombine& C,
    const int4* desc, const int4* kr, int nitems, int* jobs, int& njob,
    int (*pos)[64], float4 (*part)[4][64]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nslab = C.H / 256;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores done
  if (tid == 0) njob = 0;
  __syncthreads();
  for (int q = tid; q < nitems * BM; q += ST_THREADS) {
    const int i = q / BM, r = q % BM;
    const int4 d = desc[i];
    if (r >= d.w) continue;
    const int seg = d.x & 1, nt = (d.x >> 1) & 0x7FFF;
    // a routed tile's rows are one expert's assignments: distinct tokens
    const int t = seg ? d.z + r : C.sorted[d.z + r] / C.topk;
    int kept = 0;
    for (int j = 0; j < C.topk; ++j) kept += C.inv[t * C.topk + j] >= 0;
    const int want = kept * C.ks + (C.y_sh ? C.ks_sh : 0);
    // relaxed device-scope count: see dec_fused_finish (a stream-K unit's
    // first item also arrives for its zero slices)
    const int inc = 1 + kr[i].z;
    if (__hip_atomic_fetch_add(C.cnt + t * nslab + nt, inc, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT) == want - inc)
      jobs[atomicAdd(&njob, 1)] = t * nslab + nt;
  }
  __syncthreads();
  const int nj = njob;
  const int g = wave >> 2, wq = wave & 3;
  const __amdgpu_buffer_rsrc_t ry = dev_rsrc(C.y);
  const __amdgpu_buffer_rsrc_t rs = dev_rsrc(C.y_sh ? C.y_sh : C.y);
  const int nr = C.topk * C.ks, nsl = nr + (C.y_sh ? C.ks_sh : 0);
  for (int u0 = 0; u0 < nj; u0 += 2) {
    const bool live = u0 + g < nj;
    const int u = live ? jobs[u0 + g] : jobs[u0];
    const int t = u / nslab, c = (u % nslab) * 256 + lane * 4;
    if (wq == 0 && lane < C.topk) pos[g][lane] = C.inv[t * C.topk + lane];
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int b = wq; b < nsl; b += 4 * DC_BATCH) {
      float4 v[DC_BATCH];
#pragma unroll
      for (int k = 0; k < DC_BATCH; ++k) {
        const int sl = min(b + k * 4, nsl - 1);
        // a dropped assignment (position -1) reads row 0 and is not added
        v[k] = sl < nr
                   ? ld_dev4(ry, (sl % C.ks) * C.kstride +
                                     (long)max(pos[g][sl / C.ks], 0) * C.H + c)
                   : ld_dev4(rs, (sl - nr) * C.kstride_sh + (long)t * C.H + c);
      }
#pragma unroll
      for (int k = 0; k < DC_BATCH; ++k) {
        const int sl = b + k * 4;
        if (sl < nsl && (sl >= nr || pos[g][sl / C.ks] >= 0)) {
          acc.x += v[k].x;
          acc.y += v[k].y;
          acc.z += v[k].z;
          acc.w += v[k].w;
        }
      }
    }
    part[g][wq][lane] = acc;
    __syncthreads();
    if (wq == 0 && live) {
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float4 p = part[g][w][lane];
        acc.x += p.x;
        acc.y += p.y;
        acc.z += p.z;
        acc.w += p.w;
      }
      if (C.out_f32) {
        *(float4*)((float*)C.out + (size_t)t * C.H + c) = acc;
      } else {
        *(uint2*)((uint16_t*)C.out + (size_t)t * C.H + c) =
            make_uint2(pk_bf16(acc.x, acc.y), pk_bf16(acc.z, acc.w));
      }
    }
    __syncthreads();  // pos and part are the next pair's
  }
}

template <int BF, int MODE, bool WNT, int BM, int BF1 = BF>
__global__ __launch_bounds__(ST_THREADS, 1) void moe_stream_dec_kernel(
    SegDesc S0, SegDesc S1, int nseg, int topk, float limit, DecFuse F,
    RouteInline RI, DecCombine C, int CB, int SK) {
  constexpr int RB = BM / 16;
  // BF1 != BF: the first segment's weights are MXFP4 and the second's FP8
  // with fp32 block scales (a DeepSeek layer's routed and shared experts in
  // one launch); a workgroup streams its MXFP4 items, then its FP8 items
  constexpr bool MIX = BF1 != BF;
  static_assert(!MIX || (BF == SF_FP4 && BF1 == SF_FP8_F32S),
                "mixed formats: MXFP4 first segment, FP8 second");
  __shared__ int mix_nf4;  // mixed: the workgroup's MXFP4 items
  static_assert(BM == 16 || BM == 32, "decode tiles are 16 or 32 rows");
  __shared__ int4 desc[ST_MAX_ITEMS];
  // per item: first K step, K steps, zero slices to write (the first item
  // of a stream-K unit that fewer than ks ranges reach), 0
  __shared__ int4 kr[ST_MAX_ITEMS];
  __shared__ int sk_n;  // stream-K: the workgroup's items
  __shared__ int rsrc[ST_MAX_ITEMS][BM];
  __shared__ float rwl[ST_MAX_ITEMS][BM];
  __shared__ __attribute__((aligned(16))) uint16_t a_hi[2][BM * SD_LS];
  __shared__ __attribute__((aligned(16))) uint16_t a_lo[MODE == 1 ? 2 : 1][MODE == 1 ? BM * SD_LS : 8];
  // the batch's routing when the launch routes it (gate/up only): per-wave
  // expert histograms, the picked ids, the sorted assignment indices, the
  // tile table, and the scan scratch with the tile count after it
  constexpr bool RTE = MODE == 0;
  static_assert(RI_MAX_ROUTE_T <= ST_WAVES, "one routed token per wave");
  __shared__ int ri_hist[RTE ? ST_WAVES : 1][RTE ? RI_MAX_E : 1];
  __shared__ int ri_ids[RTE ? RI_MAX_N : 1];
  // workgroup 0: the weights of the picks routed here (up to 8 tokens of
  // at most 64 picks, one wave each), for the sorted-position table
  __shared__ float ri_w[RTE ? RI_MAX_ROUTE_T * 64 : 1];
  __shared__ int ri_sorted[RTE ? RI_MAX_N : 1];
  __shared__ __attribute__((aligned(16))) int ri_tiles[RTE ? 4 * RI_MAX_TILES : 4];
  __shared__ int ri_sh[ST_WAVES + 1];

  constexpr int NTW = MODE == 0 ? 128 : 256;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, lc = lane & 15;

  // ---- the batch's routing and permutation (RouteInline): every
  // workgroup computes the same tables in LDS; workgroup 0 also writes
  // them out ---------------------------------------------------------------
  bool inl = false;
  if constexpr (RTE) {
    if (RI.logits || RI.ids_in) {
      inl = true;
      const bool lead = blockIdx.x == 0;
      const int k = RI.topk;
      if (RI.logits) {
        // wave w routes token w; other workgroups read the rows meanwhile:
        // no write-back of the summed slices (store false)
        if (wave < RI.T) {
          if (RI.grouped) {
            // scratch: the wave's histogram row, unused until the permutation
            static_assert(2 * RI_MAX_E_GROUPED <= RI_MAX_E, "grouped routing scratch");
            float* scr = (float*)ri_hist[wave];
            route_grouped_token<RI_MAX_E_GROUPED / 64>(
                RI.logits + (size_t)wave * RI.E, RI.ks, (long)RI.T * RI.E,
                false, RI.E, k, RI.n_group, RI.topk_group, RI.scoring,
                RI.route_scale, RI.bias, scr, scr + RI_MAX_E_GROUPED,
                lead ? RI.w + (size_t)wave * k : nullptr,
                lead ? RI.ids + (size_t)wave * k : nullptr, ri_ids + wave * k,
                lead ? ri_w + wave * k : nullptr);
          } else {
            route_softmax_token<8, 2>(RI.logits + (size_t)wave * RI.E, RI.ks,
                                      (long)RI.T * RI.E, RI.E, k, RI.eps,
                                      lead ? RI.w + (size_t)wave * k : nullptr,
                                      lead ? RI.ids + (size_t)wave * k : nullptr,
                                      ri_ids + wave * k, RI.bias, false,
                                      lead ? ri_w + wave * k : nullptr);
          }
          if (lead && RI.gate && lane == 0) route_gate_finish(RI.gate, RI.T, wave, RI.ks);
        }
      } else {
        for (int i = tid; i < RI.T * k; i += ST_THREADS) ri_ids[i] = RI.ids_in[i];
      }
      __syncthreads();
      const PermDst out = lead ? PermDst{RI.counts, RI.offsets, RI.sorted,
                                         RI.inv, RI.tiles, RI.ntiles,
                                         RI.rw_sorted}
                               : PermDst{};
      const PermDst mine{nullptr, nullptr, ri_sorted, nullptr, ri_tiles,
                         &ri_sh[ST_WAVES]};
      // (the batches routed here; the table is not asked for otherwise)
      const float* w_src = lead && RI.rw_sorted && RI.logits ? ri_w : nullptr;
      // a batch routed here (distinct experts per token) of at most bm
      // tokens and 64 assignments: one tile per expert, sorted in one wave
      if (RI.logits && RI.T <= RI.bm && RI.T * k <= 64)
        permute_small_wave(ri_ids, RI.T * k, RI.E, RI.max_tiles, out, mine,
                           (uint32_t*)ri_hist[0], w_src);
      else
        permute_block<ST_WAVES, RI_G, RI_MAX_E>(ri_ids, RI.T * k, RI.E, RI.nbits,
                                                 RI.bm, RI.max_tiles, out, mine,
                                                 ri_hist, ri_sh, nullptr, 0, w_src);
      __syncthreads();
    }
  }
  // the routed segment's tile table and sorted rows: this launch's own or
  // the permutation launch's
  const int* tiles0 = inl ? ri_tiles : S0.tile_info;
  const int* sorted0 = inl ? ri_sorted : S0.sorted_idx;

  // Units: a row tile's column slab of a segment (routed units first, then
  // the shared expert's). Items: K steps [kb0, kb0 + nkb) of a unit, whose
  // partial sums go to K slice `slot` (desc.x bits 16-30; kr).
  auto seg_units = [&](const SegDesc& S, bool own) {
    const int rt = own ? ri_sh[ST_WAVES]
                 : S.tile_info ? *S.num_tiles : (S.total_rows + BM - 1) / BM;
    return rt * (S.N / NTW);
  };
  const int nu0 = seg_units(S0, inl);
  const int nu1 = nseg > 1 ? seg_units(S1, false) : 0;
  const int nx = gridDim.x / 8;
  const int xcd = blockIdx.x % 8, jx = blockIdx.x / 8;
  // item idx := unit li of segment seg, K steps [kb0, kb0 + nkb), slice slot
  auto make_item = [&](int idx, int seg, int li, int kb0, int nkb, int slot,
                       int fill) {
    const SegDesc& S = seg ? S1 : S0;
    const int ntn = S.N / NTW;
    const int rt = li / ntn, nt = li % ntn;
    int e = 0, rb, rows;
    const int* ti = seg ? S.tile_info : tiles0;
    if (ti) {
      const int4 d = *(const int4*)(ti + 4 * rt);
      e = d.x;
      rb = d.y;
      rows = min(BM, d.z);
    } else {
      rb = rt * BM;
      rows = min(BM, S.total_rows - rb);
    }
    // x: segment (bit 0), column slab (bits 1-15), K slice (bits 16-30)
    desc[idx] = make_int4(seg | (nt << 1) | (slot << 16), e, rb, rows);
    kr[idx] = make_int4(kb0, nkb, fill, 0);
  };
  int nitems;
  if (SK) {
    // stream-K: this workgroup's range of the units' cost line (sk_lreq);
    // the ranges of an XCD are adjacent, so that a tile's units meet in
    // its L2. The MXFP4 units come first on the line: so do their items.
    // 32-bit arithmetic: the host bounds the line's cost times the grid
    // below 2^31 (go_stream_dec).
    using U = uint32_t;
    constexpr U W1 = MIX ? 2 : 1;
    const U KB0 = S0.K / 128, KB1 = nseg > 1 ? S1.K / 128 : 1;
    const U c0 = KB0, c1 = KB1 * W1, cs = (U)nu0 * c0;
    const U C = cs + (U)nu1 * c1;
    U lreq = sk_lreq<U>(KB0, 1, S0.ksplit);
    if (nseg > 1) lreq = max(lreq, sk_lreq<U>(KB1, W1, S1.ksplit));
    const U G = sk_ranges<U>(C, lreq, gridDim.x);
    const U r = (U)xcd * nx + jx;
    if (C == 0 || r >= G) return;
    const U a = r * C / G, b = (r + 1) * C / G;
    auto unit_of = [&](U c) { return c < cs ? c / c0 : nu0 + (c - cs) / c1; };
    const U ua = unit_of(a), ncand = unit_of(b - 1) - ua + 1;
    if (ncand > 64) {  // more units than a wave's lanes: a sizing error
      if (tid == 0) stream_item_overflow = 1;
      return;
    }
    if (wave == 0) {
      bool live = false;
      int seg = 0, li = 0, kb0 = 0, nkb = 0, slot = 0, fill = 0;
      if ((U)lane < ncand) {
        const U u = ua + lane;
        seg = u >= (U)nu0;
        li = (int)(seg ? u - nu0 : u);
        const U KB = seg ? KB1 : KB0, w = seg ? W1 : 1;
        const int ks = seg ? S1.ksplit : S0.ksplit;
        const U cu = seg ? cs + (U)li * c1 : (U)li * c0;
        // the unit's steps whose start cu + j w lies in [a, b) (b > cu:
        // the unit starts before the range ends)
        const U jlo = a <= cu ? 0 : (a - cu + w - 1) / w;
        const U jhi = min(KB, (b - cu + w - 1) / w);
        live = jlo < jhi;
        // range of a cost position: the r with r C / G <= c < (r + 1) C / G
        auto range_of = [&](U c) { return ((c + 1) * G - 1) / C; };
        const U rfirst = range_of(cu);
        const int nsl = (int)(range_of(cu + (KB - 1) * w) - rfirst + 1);
        slot = (int)r - (int)rfirst;
        fill = slot == 0 ? ks - nsl : 0;
        kb0 = (int)jlo;
        nkb = (int)jhi - (int)jlo;
      }
      const uint64_t lm = __ballot(live);
      const int idx = __popcll(lm & ((1ull << lane) - 1));
      if (live && idx < ST_MAX_ITEMS) make_item(idx, seg, li, kb0, nkb, slot, fill);
      const uint64_t f8 = __ballot(live && seg);
      if (lane == 0) {
        sk_n = __popcll(lm);
        if constexpr (MIX) mix_nf4 = __popcll(lm) - __popcll(f8);
      }
    }    __syncthreads();
    nitems = sk_n;
  } else {
    // XCD x takes chunks x, x + 8, ... of CB items (a row tile's items, its
    // column slabs and K chunks, at most: dec_deal_chunk), so that every
    // XCD gets the same mix of routed and shared-expert items (as in the
    // prefill kernel; C3 B=32 163.1 / 164.2 -> 161.6 / 160.6 us, B=1 and
    // B=8 unchanged) (the host sizes the grid for this deal: stream_dec_grid)
    const int n0 = nu0 * S0.ksplit;
    const int total = n0 + nu1 * (nseg > 1 ? S1.ksplit : 1);
    const int ncf = total / CB, crem = total % CB;
    const int xcount = (ncf > xcd ? (ncf - xcd + 7) / 8 : 0) * CB + (ncf % 8 == xcd ? crem : 0);
    nitems = xcount > jx ? (xcount - jx + nx - 1) / nx : 0;
    if (nitems <= ST_MAX_ITEMS && tid < nitems) {
      const int qx = jx + tid * nx;  // the XCD's qx-th item
      const int it = (xcd + 8 * (qx / CB)) * CB + qx % CB;
      const int seg = it >= n0;
      const SegDesc& S = seg ? S1 : S0;
      const int li = seg ? it - n0 : it;
      const int kc = li % S.ksplit, KB = S.K / 128;
      const int kb0 = kc * KB / S.ksplit;
      int idx = tid;
      if constexpr (MIX) {  // MXFP4 (first-segment) items first, in deal order
        static_assert(ST_MAX_ITEMS <= 64, "a workgroup's items are one wave's lanes");
        const uint64_t fp8 = __ballot(seg);  // lanes tid < nitems <= 32 of wave 0
        const int nf8_below = __popcll(fp8 & ((1ull << tid) - 1));
        const int nf4 = nitems - __popcll(fp8);
        idx = seg ? nf4 + nf8_below : tid - nf8_below;
        if (tid == 0) mix_nf4 = nf4;
      }
      make_item(idx, seg, li / S.ksplit, kb0, (kc + 1) * KB / S.ksplit - kb0, kc, 0);
    }
  }
  if (nitems > ST_MAX_ITEMS) {  // host sizes the grid: a sizing error
    if (tid == 0) stream_item_overflow = 1;
    return;
  }
  if (nitems == 0) return;

  __syncthreads();
  for (int q = tid; q < nitems * BM; q += ST_THREADS) {
    const int i = q / BM, r = q % BM;
    const int4 d = desc[i];
    const SegDesc& S = (d.x & 1) ? S1 : S0;
    int src = 0;
    float rw = 1.f;
    if (r < d.w) {
      const int p = d.z + r;
      const int* si = (d.x & 1) ? S.sorted_idx : sorted0;
      src = S.gather ? si[p] / topk : p;
      if (S.row_w) rw = S.row_w[S.row_w_by_idx ? si[p] : p];
    }
    rsrc[i][r] = src;
    rwl[i][r] = rw;
  }
  __syncthreads();

  // K steps [kb0, kb0 + nkb) of item i
  auto kchunk = [&](int i, int& kb0, int& nkb) {
    kb0 = kr[i].x;
    nkb = kr[i].y;
  };

  // activation tile of a K step: BM rows x 128 values; thread tid takes
  // rows tid / 32 + 16 r and values [4 (tid % 32), +4)
  const int a_row = tid >> 5, a_col = (tid & 31) * 4;
  typedef typename std::conditional<MODE == 0, u32x2, v4uv>::type AVec;
  struct ASet {
    AVec v[RB];
  };
  struct BSetD {
    v8i v[2];
    uint32_t sc;
    float sb0, sb1;
  };

  f32x4 acc[RB][2];
  auto clear_acc = [&]() {
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r][0] = acc[r][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
  };
  clear_acc();

  // acc[r][s][v]: row 16 r + lc of the tile, output column 4 lg + v of
  // subtile s
  // (slices [ks - fill, ks) of a stream-K unit no range reached: zeros)
  auto epilogue = [&](int i) {
    const int4 d = desc[i];
    const int seg = d.x & 1, nt = (d.x >> 1) & 0x7FFF, kc = d.x >> 16;
    const SegDesc& S = seg ? S1 : S0;
    const int fill = kr[i].z;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int row = 16 * r + lc;
      if (row >= d.w) continue;  // K chunk kc's slice (kc = 0 unsplit)
      const float rw = rwl[i][row];
      if constexpr (MODE == 0) {
        if (S.ksplit > 1) {  // chunk sums; SwiGLU in the finish
          const long og = kc * S.pstride + (long)(d.z + row) * S.N +
                          nt * 128 + wave * 16 + lg * 4;
          float* pg = S.pp + og;
          float* pu = pg + S.ksplit * S.pstride;
          const long o0 = og - kc * S.pstride;  // slice 0
          if (F.cnt) {
            const __amdgpu_buffer_rsrc_t rp = dev_rsrc(S.pp);
            st_dev4(rp, og, acc[r][0][0], acc[r][0][1], acc[r][0][2], acc[r][0][3]);
            st_dev4(rp, og + S.ksplit * S.pstride, acc[r][1][0], acc[r][1][1],
                    acc[r][1][2], acc[r][1][3]);
            for (int z = S.ksplit - fill; z < S.ksplit; ++z) {
              st_dev4(rp, o0 + z * S.pstride, 0.f, 0.f, 0.f, 0.f);
              st_dev4(rp, o0 + (S.ksplit + z) * S.pstride, 0.f, 0.f, 0.f, 0.f);
            }
          } else {
            *(float4*)pg = make_float4(acc[r][0][0], acc[r][0][1], acc[r][0][2], acc[r][0][3]);
            *(float4*)pu = make_float4(acc[r][1][0], acc[r][1][1], acc[r][1][2], acc[r][1][3]);
            for (int z = S.ksplit - fill; z < S.ksplit; ++z) {
              *(float4*)(S.pp + o0 + z * S.pstride) = make_float4(0.f, 0.f, 0.f, 0.f);
              *(float4*)(S.pp + o0 + (S.ksplit + z) * S.pstride) =
                  make_float4(0.f, 0.f, 0.f, 0.f);
            }
          }
          continue;
        }
        float h[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float g = acc[r][0][v], u = acc[r][1][v];
          if (limit > 0.f) {
            u = fminf(fmaxf(u, -limit), limit);
            g = fminf(g, limit);
          }
          h[v] = silu_f32(g) * u * rw;
        }
        float* out = (float*)S.hq + (size_t)(d.z + row) * S.N + nt * 128 + wave * 16 + lg * 4;
        *(float4*)out = make_float4(h[0], h[1], h[2], h[3]);
      } else {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const long o0 = (long)(d.z + row) * S.N + nt * 256 + wave * 32 +
                          sb * 16 + lg * 4;
          const long o = kc * S.pstride + o0;
          if (C.cnt) {  // read by the fused combine's finisher: device scope
            const __amdgpu_buffer_rsrc_t ry = dev_rsrc((const float*)S.y);
            st_dev4(ry, o, acc[r][sb][0] * rw, acc[r][sb][1] * rw,
                    acc[r][sb][2] * rw, acc[r][sb][3] * rw);
            for (int z = S.ksplit - fill; z < S.ksplit; ++z)
              st_dev4(ry, o0 + z * S.pstride, 0.f, 0.f, 0.f, 0.f);
          } else {
            *(float4*)((float*)S.y + o) =
                make_float4(acc[r][sb][0] * rw, acc[r][sb][1] * rw,
                            acc[r][sb][2] * rw, acc[r][sb][3] * rw);
            for (int z = S.ksplit - fill; z < S.ksplit; ++z)
              *(float4*)((float*)S.y + o0 + z * S.pstride) = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
      }
    }
    clear_acc();
  };

  // The streamed K steps of items [i0, i1), whose weights are all MXFP4
  // (F4: 16 KB weight blocks, e8m0 scales applied in the conversion) or all
  // FP8 (32 KB blocks, the step's partial times its fp32 block scale): one
  // format per pipeline, so that its loads keep three steps in flight (a
  // per-step format branch left the compiler waiting on all but a few
  // loads at every step)
  auto pipeline = [&](auto f4c, const int i0, const int i1) {
    constexpr bool F4 = decltype(f4c)::value;
    int total_steps = 0;
    for (int i = i0; i < i1; ++i) {
      int kb0, nkb;
      kchunk(i, kb0, nkb);
      total_steps += nkb;
    }

    int pi = i0, pkb = 0, pKB = 1;
    const uint8_t* pa[RB];
    const uint8_t* pb = nullptr;
    const float *ps0 = nullptr, *ps1 = nullptr;
    const uint16_t* ps4 = nullptr;
    auto p_enter = [&](int i) {
      const int4 d = desc[i];
      const int seg = d.x & 1, nt = (d.x >> 1) & 0x7FFF;
      const SegDesc& S = seg ? S1 : S0;
      const int K = S.K, KB = K / 128, N = S.N, NT = N / NTW;
      int kb0;
      kchunk(i, kb0, pKB);
#pragma unroll
      for (int r = 0; r < RB; ++r)
        pa[r] = S.a + ((size_t)rsrc[i][a_row + 16 * r] * K + kb0 * 128 + a_col) *
                          (MODE == 0 ? 2 : 4);
      const size_t blk0 = ((size_t)d.y * NT + nt) * KB + kb0;
      if constexpr (F4) {
        pb = S.wp + blk0 * 16384 + (wave * 2) * 1024 + lane * 16;
        ps4 = (const uint16_t*)S.s0 + blk0 * 512 + wave * 64 + lane;
      } else {
        pb = S.wp + blk0 * 32768 + (wave * 4) * 1024 + lane * 16;
        if constexpr (MODE == 0) {
          ps0 = (const float*)S.s0 + blk0;
          ps1 = (const float*)S.s1 + blk0;
        } else {
          const int nblk = nt * 2 + wave / 4;
          ps0 = ps1 = (const float*)S.s0 + ((size_t)d.y * (N / 128) + nblk) * KB + kb0;
        }
      }
    };
    auto p_advance = [&]() {
      if (pkb + 1 < pKB) {
        ++pkb;
      } else if (pi + 1 < i1) {
        ++pi;
        pkb = 0;
        p_enter(pi);
      }
    };
    auto prefetch = [&](ASet& af, BSetD& b) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
        af.v[r] = *(const AVec*)(pa[r] + (size_t)pkb * 128 * (MODE == 0 ? 2 : 4));
      const uint8_t* base = pb + (size_t)pkb * (F4 ? 16384 : 32768);
      if constexpr (F4) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const uint4 v = ld_stream<WNT>(base + s * 1024);
          b.v[s] = (v8i){(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
        }
        b.sc = __builtin_nontemporal_load(ps4 + (size_t)pkb * 512);
        b.sb0 = b.sb1 = 1.f;
      } else {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const uint4 lo4 = ld_stream<WNT>(base + (2 * s) * 1024);
          const uint4 hi4 = ld_stream<WNT>(base + (2 * s + 1) * 1024);
          b.v[s] = (v8i){(int)lo4.x, (int)lo4.y, (int)lo4.z, (int)lo4.w,
                         (int)hi4.x, (int)hi4.y, (int)hi4.z, (int)hi4.w};
        }
        b.sc = 0;
        b.sb0 = ps0[pkb];
        b.sb1 = MODE == 0 ? ps1[pkb] : b.sb0;
      }
      p_advance();
    };

    int ci = i0, ckb = 0, cKB = 1, crows = 0;
    auto c_enter = [&](int i) {
      int kb0;
      kchunk(i, kb0, cKB);
      crows = desc[i].w;
    };

    auto step = [&](int st, ASet& acur, ASet& aload, BSetD& bcur, BSetD& bload) {
      const int buf = st & 1;
#pragma unroll
      for (int r = 0; r < RB; ++r) {  // activations -> LDS as bf16 (mode 1: hi
                                      // and lo halves), rows past the tile zeroed
        const int row = a_row + 16 * r;
        const uint32_t m = row < crows ? ~0u : 0u;
        if constexpr (MODE == 0) {
          *(u32x2*)(a_hi[buf] + row * SD_LS + a_col) =
              (u32x2){acur.v[r].x & m, acur.v[r].y & m};
        } else {
          float f[4] = {__uint_as_float(acur.v[r].x & m), __uint_as_float(acur.v[r].y & m),
                        __uint_as_float(acur.v[r].z & m), __uint_as_float(acur.v[r].w & m)};
          uint32_t hb[4], lb[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            hb[j] = f32_to_bf16(f[j]);
            lb[j] = f32_to_bf16(f[j] - __uint_as_float(hb[j] << 16));
          }
          *(u32x2*)(a_hi[buf] + row * SD_LS + a_col) =
              (u32x2){hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
          *(u32x2*)(a_lo[buf] + row * SD_LS + a_col) =
              (u32x2){lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)};
        }
      }
      __syncthreads();
      prefetch(aload, bload);
      f32x4 part[RB][2];
#pragma unroll
      for (int r = 0; r < RB; ++r) part[r][0] = part[r][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const int ko = lg * 32 + mm * 8;
        bf16x8 xh[RB], xl[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          xh[r] = *(const bf16x8*)(a_hi[buf] + (16 * r + lc) * SD_LS + ko);
          if constexpr (MODE == 1) xl[r] = *(const bf16x8*)(a_lo[buf] + (16 * r + lc) * SD_LS + ko);
        }
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          bf16x8 wv;
          if constexpr (F4) {
            wv = fp4x8_to_bf16((uint32_t)bcur.v[sb][mm], (bcur.sc >> (8 * sb)) & 0xFFu);
          } else {
            wv = fp8x8_to_bf16((uint32_t)bcur.v[sb][2 * mm], (uint32_t)bcur.v[sb][2 * mm + 1]);
          }
#pragma unroll
          for (int r = 0; r < RB; ++r) {
            f32x4& tgt = F4 ? acc[r][sb] : part[r][sb];
            tgt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, xh[r], tgt, 0, 0, 0);
            if constexpr (MODE == 1)
              tgt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, xl[r], tgt, 0, 0, 0);
          }
        }
      }
      if constexpr (!F4) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            acc[r][0][v] = fmaf(part[r][0][v], bcur.sb0, acc[r][0][v]);
            acc[r][1][v] = fmaf(part[r][1][v], bcur.sb1, acc[r][1][v]);
          }
      }
      if (++ckb == cKB) {
        epilogue(ci);
        ckb = 0;
        if (ci + 1 < i1) c_enter(++ci);
      }
    };

    // NS register sets per operand, prefetch distance NS - 1
    constexpr int NS = F4 ? DEC_SETS_F4 : DEC_SETS_F8;
    BSetD bs[NS];
    ASet as[NS];
    p_enter(i0);
    c_enter(i0);
#pragma unroll
    for (int j = 0; j + 1 < NS; ++j) prefetch(as[j], bs[j]);
    int st = 0;
    for (; st + NS <= total_steps; st += NS) {
#pragma unroll
      for (int j = 0; j < NS; ++j)
        step(st + j, as[j], as[(j + NS - 1) % NS], bs[j], bs[(j + NS - 1) % NS]);
    }
#pragma unroll
    for (int j = 0; j + 1 < NS; ++j)
      if (st + j < total_steps)
        step(st + j, as[j], as[(j + NS - 1) % NS], bs[j], bs[(j + NS - 1) % NS]);
  };
  if constexpr (MIX) {
    // the MXFP4 items were placed first; the barrier hands the LDS
    // activation buffers from the last MXFP4 step to the first FP8 one
    const int nf4 = mix_nf4;
    if (nf4 > 0) pipeline(std::true_type{}, 0, nf4);
    if (nf4 < nitems) {
      if (nf4 > 0) __syncthreads();
      pipeline(std::false_type{}, nf4, nitems);
    }
  } else {
    pipeline(std::integral_constant<bool, BF == SF_FP4>{}, 0, nitems);
  }
  if constexpr (MODE == 0) {
    if (F.cnt) {
      __shared__ int jobs[ST_MAX_ITEMS];
      __shared__ int njob;
      dec_fused_finish<BM>(S0, S1, limit, F, desc, kr, nitems, jobs, njob);
    }
  } else {
    if (C.cnt) {
      __shared__ int cjobs[ST_MAX_ITEMS * BM];
      __shared__ int ncj;
      __shared__ int cpos[2][64];
      __shared__ float4 cpart[2][4][64];
      dec_fused_combine<BM>(S0, S1, C, desc, kr, nitems, cjobs, ncj, cpos, cpart);
    }
  }
}

static int num_cus() {
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

// Decode K split. A launch's items (upper_items at most) of KB K steps each
// are cut into ks chunks and dealt over the persistent grid (G workgroups,
// #CUs rounded up to a multiple of 8); its time goes with the largest
// number of K steps one workgroup streams, ceil(items ks / G) ceil(KB / ks).
// Few long items (one expert: a dense MLP, a single token) would leave most
// CUs idle, and equal items that do not divide evenly over the grid leave a
// tail (136 items of 40 steps: 40 steps unsplit, 30 at ks = 4, 24 at 5).
static long dec_split_steps(long items, int KB, int ks) {
  const long G = 8L * ((num_cus() + 7) / 8);
  return (items * ks + G - 1) / G * ((KB + ks - 1) / ks);
}

// The ks in [1, cap] of fewest steps, each split charged `extra` steps and
// required to save at least `min_gain` of the unsplit steps (ties: smaller).
static int dec_best_split(long items, int KB, int cap, long extra,
                          double min_gain) {
  const long base = dec_split_steps(items, KB, 1);
  int best = 1;
  long bcost = base;
  for (int ks = 2; ks <= cap; ++ks) {
    const long c = dec_split_steps(items, KB, ks) + extra;
    if (c < bcost && c <= (1.0 - min_gain) * base) {
      best = ks;
      bcost = c;
    }
  }
  return best;
}

constexpr long DEC_TARGET_ITEMS = 512;
constexpr int DEC_MAX_KSPLIT = 32;
// a finish launch costs about as much as streaming three K steps per CU
constexpr long DEC_FINISH_STEPS = 3;

// Gate/up: only launches with fewer than two items per CU (upper_items is
// a bound from the tile count, well above the routed count at larger
// batches), into chunks of at least four K steps, at most 8 (the finish
// reads every slice).
int dec_ksplit_up(long upper_items, int KB) {
  if (upper_items <= 0 || upper_items >= DEC_TARGET_ITEMS) return 1;
  return dec_best_split(upper_items, KB, std::max(1, std::min(KB / 4, 8)),
                        DEC_FINISH_STEPS, 0.0);
}

// The largest number of K steps a workgroup of a chunk-dealt decode launch
// streams (chunks of a routed row tile's items to the XCDs in turn, dealt
// round-robin over an XCD's workgroups; dec_deal_chunk, stream_dec_grid)
// when its items, exp_items of them routed as expected (the chunk and the
// grid follow the launch's bound upper_items), are cut into ks K chunks.
static long dec_dealt_items(long exp_items, long upper_items, long tile_items,
                            int ks) {
  const long n = exp_items * ks, nu = upper_items * ks;
  const long cb = std::max(1L, std::min(tile_items * ks, nu / 64));
  const long nx = stream_dec_grid(nu, num_cus(), cb, ST_MAX_ITEMS) / 8;
  return (chunked_xcd_share(n, cb) + nx - 1) / nx;
}
static long dec_dealt_steps(long exp_items, long upper_items, long tile_items,
                            int KB, int ks) {
  return dec_dealt_items(exp_items, upper_items, tile_items, ks) *
         ((KB + ks - 1) / ks);
}

// a split (its finish launch, or the fused finish's slice reads) costs
// about four K steps of the launch
constexpr long DEC_FINISH_STEPS_DEALT = 4;

int dec_ksplit_up_dealt(long upper_items, long exp_items, long tile_items,
                        int KB) {
  if (upper_items <= 0 || upper_items >= DEC_TARGET_ITEMS_DEALT) return 1;
  const int cap = std::max(1, std::min(KB / 4, 8));
  int best = 1;
  long bcost = dec_dealt_steps(exp_items, upper_items, tile_items, KB, 1);
  for (int ks = 2; ks <= cap; ++ks) {
    const long c = dec_dealt_steps(exp_items, upper_items, tile_items, KB, ks) +
                   DEC_FINISH_STEPS_DEALT;
    if (c < bcost) {
      best = ks;
      bcost = c;
    }
  }
  return best;
}

// Down launches dealt the same way: no finish (the combine adds the
// slices), but every item costs about one K step beyond its own (its
// prologue and y stores; at C3 the items are 4 K steps long).
int dec_ksplit_dealt(long upper_items, long exp_items, long tile_items, int KB) {
  if (upper_items <= 0 || KB <= 1) return 1;
  int best = 1;
  long bcost = dec_dealt_items(exp_items, upper_items, tile_items, 1) * (KB + 1);
  for (int ks = 2; ks <= std::min(KB, DEC_MAX_KSPLIT); ++ks) {
    const long c = dec_dealt_items(exp_items, upper_items, tile_items, ks) *
                   ((KB + ks - 1) / ks + 1);
    if (c < bcost) {
      best = ks;
      bcost = c;
    }
  }
  return best;
}

// h = silu(g) * u from the K-chunk slices of split mode-0 segments, rows
// [0, total_rows) of each. A thread takes four columns of one row: all of
// its 2 ks slice loads are issued together, then added in chunk order.
constexpr int SF_MAX_KS = 8;

__global__ __launch_bounds__(256) void split_finish_kernel(SegDesc S0,
                                                           SegDesc S1, int nseg,
                                                           float limit) {
  const long n0 = (long)S0.total_rows * S0.N / 4;
  const long n1 = nseg > 1 ? (long)S1.total_rows * S1.N / 4 : 0;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n0 + n1) return;
  const bool second = i >= n0;
  const SegDesc& S = second ? S1 : S0;
  const long j = (second ? i - n0 : i) * 4;
  const int ks = S.ksplit;
  float4 g[SF_MAX_KS], u[SF_MAX_KS];
#pragma unroll
  for (int q = 0; q < SF_MAX_KS; ++q) {
    const int qq = min(q, ks - 1);
    g[q] = *(const float4*)(S.pp + qq * S.pstride + j);
    u[q] = *(const float4*)(S.pp + (ks + qq) * S.pstride + j);
  }
  float gs[4] = {0.f, 0.f, 0.f, 0.f}, us[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < SF_MAX_KS; ++q) {
    if (q < ks) {
      gs[0] += g[q].x; gs[1] += g[q].y; gs[2] += g[q].z; gs[3] += g[q].w;
      us[0] += u[q].x; us[1] += u[q].y; us[2] += u[q].z; us[3] += u[q].w;
    }
  }
  float h[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float gv = gs[v], uv = us[v];
    if (limit > 0.f) {
      uv = fminf(fmaxf(uv, -limit), limit);
      gv = fminf(gv, limit);
    }
    h[v] = silu_f32(gv) * uv;
  }
  *(float4*)((float*)S.hq + j) = make_float4(h[0], h[1], h[2], h[3]);
}

int launch_split_finish(const SegDesc& s0, const SegDesc* s1, float limit,
                        hipStream_t st) {
  long n = 0;
  for (const SegDesc* s : {&s0, s1}) {
    if (!s) continue;
    SLLM_REQUIRE(s->pp && s->hq && s->ksplit >= 1 && s->ksplit <= SF_MAX_KS &&
                     s->N % 4 == 0 && s->total_rows > 0 &&
                     s->pstride >= (long)s->total_rows * s->N,
                 "split finish: bad segment (rows=%d N=%d ks=%d)",
                 s->total_rows, s->N, s->ksplit);
    n += (long)s->total_rows * s->N / 4;
  }
  SLLM_REQUIRE(n < (1L << 31) * 256, "split finish: too large");
  split_finish_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
      s0, s1 ? *s1 : s0, s1 ? 2 : 1, limit);
  SLLM_LAUNCHED();
  return 0;
}

long dec_launch_grid(long upper_items, long chunk) {
  return stream_dec_grid(upper_items, num_cus(), chunk, ST_MAX_ITEMS);
}

// Down: the combine adds the slices, so a split costs no launch; it must
// save a fifth of the steps (the bound overstates routed items).
int dec_ksplit(long upper_items, int KB) {
  if (upper_items <= 0 || KB <= 1) return 1;
  return dec_best_split(upper_items, KB, std::min(KB, DEC_MAX_KSPLIT), 0, 0.2);
}

// Stream-K launches. Items a workgroup can receive: a range of length L
// (at most ceil(C / grid), or under 2 lreq where the ranges are made
// longer) meets at most ceil(L / cmin) + 1 units.
static long sk_items_bound(long cbound, long grid, long cmin, long lreq) {
  const long l = std::max((cbound + grid - 1) / grid, 2 * lreq);
  return (l + cmin - 1) / cmin + 1;
}

// The grid of a stream-K launch over a cost line of at most cbound: the
// device's CUs (a multiple of 8), grown until no workgroup can receive
// more than ST_MAX_ITEMS items; 0 when the ranges' least length alone
// exceeds that.
static long sk_grid(long cbound, long cmin, long lreq) {
  if (sk_items_bound(0, 1, cmin, lreq) > ST_MAX_ITEMS) return 0;
  long grid = 8L * ((num_cus() + 7) / 8);
  while (sk_items_bound(cbound, grid, cmin, lreq) > ST_MAX_ITEMS) grid += 8;
  return grid;
}

long dec_sk_launch_grid(int nseg, const long* units, const int* KB,
                        const int* w, const int* ks) {
  long cbound = 0, cmin = 0, lreq = 1;
  for (int i = 0; i < nseg; ++i) {
    if (ks[i] < 2 || ks[i] > KB[i]) return 0;
    const long cu = (long)KB[i] * w[i];
    cbound += units[i] * cu;
    cmin = i ? std::min(cmin, cu) : cu;
    lreq = std::max(lreq, sk_lreq(KB[i], w[i], ks[i]));
  }
  return sk_grid(cbound, cmin, lreq);
}

bool dec_sk_plan(int nseg, const long* units, const int* KB, const int* w,
                 int cap, int* ks) {
  long cbound = 0, cmin = 0, lreq = 1;
  for (int i = 0; i < nseg; ++i) cbound += units[i] * KB[i] * w[i];
  if (cbound <= 0) return false;
  // a range of the expected length (the tile bound overstates the routed
  // tiles: 5/8 of it) spans each unit in ks_i slices
  const long G0 = 8L * ((num_cus() + 7) / 8);
  const long lest = std::max(1L, cbound * 5 / (8 * G0));
  for (int i = 0; i < nseg; ++i) {
    const long need = ((long)(KB[i] - 1) * w[i] + lest - 1) / lest + 1;
    ks[i] = (int)std::max(2L, std::min((long)std::min(cap, KB[i]), need));
    if (ks[i] < 2) return false;  // one K step: nothing to split
    const long cu = (long)KB[i] * w[i];
    cmin = i ? std::min(cmin, cu) : cu;
    lreq = std::max(lreq, sk_lreq(KB[i], w[i], ks[i]));
  }
  return sk_grid(cbound, cmin, lreq) > 0;
}


// Host bound of a launch's item count: per segment, (row tiles: the tile
// table's bound, or ceil(total_rows / bm) for identity rows) x column slabs
// x K chunks. Refuses (rc -2) a caller's upper_items below it, since the grid
// sized from upper_items could then deal a workgroup more than ST_MAX_ITEMS.
static int check_item_bound(const SegDesc& s0, const SegDesc* s1, int ntw,
                            int bm, long upper_items, const char* who) {
  long bound = 0;
  for (const SegDesc* s : {&s0, s1}) {
    if (!s) continue;
    SLLM_REQUIRE(!s->tile_info || s->max_tiles > 0,
                 "%s: a tile-table segment needs its max_tiles bound", who);
    const long rt = s->tile_info ? s->max_tiles : (s->total_rows + bm - 1) / bm;
    bound += rt * (s->N / ntw) * std::max(1, s->ksplit);
  }
  SLLM_CAPACITY(upper_items >= bound,
                "%s: upper_items %ld below the item bound %ld", who,
                upper_items, bound);
  return 0;
}

// upper_items: an upper bound of the total item count (sizes the grid so
// that no workgroup receives more than ST_MAX_ITEMS items).
template <int BF, int MODE>
static int go_stream(const SegDesc& s0, const SegDesc* s1, int topk,
                     float limit, int pow2, long upper_items, hipStream_t st) {
  const bool perstep = s0.K % 512 != 0 || (s1 && s1->K % 512 != 0);
  {
    const int rc = check_item_bound(s0, s1, MODE == 0 ? 128 : 256, ST_BM,
                                    upper_items, "stream gemm");
    if (rc) return rc;
  }
  // one workgroup per CU: a workgroup with more than ST_MAX_ITEMS items
  // takes them in chunks
  const long grid = stream_grid(upper_items, num_cus(), 1 << 30);
  SLLM_REQUIRE(grid < (1L << 31), "stream gemm: grid too large");
  SegDesc dummy = s0;
  const SegDesc& b = s1 ? *s1 : dummy;
  const int ns = s1 ? 2 : 1;
  const bool nt = !s0.wreuse;
  if (perstep && nt)
    moe_stream_kernel<BF, MODE, true, true><<<(unsigned)grid, ST_THREADS, 0, st>>>(
        s0, b, ns, topk, limit, pow2);
  else if (perstep)
    moe_stream_kernel<BF, MODE, true, false><<<(unsigned)grid, ST_THREADS, 0, st>>>(
        s0, b, ns, topk, limit, pow2);
  else if (nt)
    moe_stream_kernel<BF, MODE, false, true><<<(unsigned)grid, ST_THREADS, 0, st>>>(
        s0, b, ns, topk, limit, pow2);
  else
    moe_stream_kernel<BF, MODE, false, false><<<(unsigned)grid, ST_THREADS, 0, st>>>(
        s0, b, ns, topk, limit, pow2);
  SLLM_LAUNCHED();
  return 0;
}

int launch_stream(int bf, int mode, const SegDesc& s0, const SegDesc* s1,
                  int topk, float limit, int pow2, long upper_items,
                  hipStream_t st) {
  SLLM_REQUIRE(bf >= 0 && bf <= 2 && (mode == 0 || mode == 1),
               "stream gemm: bad format");
  const int ntw = mode == 0 ? 128 : 256;
  for (const SegDesc* s : {&s0, s1}) {
    if (!s) continue;
    SLLM_REQUIRE(s->a && s->sa && s->wp && s->s0 && s->N % ntw == 0 &&
                     s->K % 128 == 0 && s->K > 0,
                 "stream gemm: bad segment (N=%d K=%d)", s->N, s->K);
    SLLM_REQUIRE(mode == 1 ? s->y != nullptr : (s->hq && s->hs),
                 "stream gemm: missing outputs");
    SLLM_REQUIRE(bf == SF_FP4 || mode == 1 || s->s1,
                 "stream gemm: missing W3 scales");
    SLLM_REQUIRE((!s->gather && !s->row_w_by_idx) || s->sorted_idx,
                 "stream gemm: gather / row_w_by_idx need sorted_idx");
  }
#define GO(B, M)                                                              \
  return go_stream<B, M>(s0, s1, topk, limit, pow2, upper_items, st)
  if (mode == 0) {
    if (bf == SF_FP8_F32S) GO(SF_FP8_F32S, 0);
    if (bf == SF_FP8_POW2) GO(SF_FP8_POW2, 0);
    GO(SF_FP4, 0);
  } else {
    if (bf == SF_FP8_F32S) GO(SF_FP8_F32S, 1);
    if (bf == SF_FP8_POW2) GO(SF_FP8_POW2, 1);
    GO(SF_FP4, 1);
  }
#undef GO
}

template <int BF, int MODE, int BM, int BF1 = BF>
static int go_stream_dec(const SegDesc& s0, const SegDesc* s1, int topk,
                         float limit, long upper_items, hipStream_t st,
                         const DecFuse& fuse, const RouteInline& route,
                         const DecCombine& comb, bool sk) {
  constexpr int NTW = MODE == 0 ? 128 : 256;
  {
    const int rc = check_item_bound(s0, s1, NTW, BM, upper_items,
                                    "stream decode gemm");
    if (rc) return rc;
  }
  long cb = 1, grid;
  if (sk) {
    // stream-K: the cost line's bound from the segments' row-tile bounds
    long un[2];
    int kb[2], w[2], ks[2];
    for (int i = 0; i < (s1 ? 2 : 1); ++i) {
      const SegDesc& s = i ? *s1 : s0;
      const long rt = s.tile_info ? s.max_tiles : (s.total_rows + BM - 1) / BM;
      SLLM_REQUIRE(s.ksplit >= 2 && s.ksplit <= s.K / 128,
                   "stream decode gemm: stream-K needs 2..K/128 slices (%d)",
                   s.ksplit);
      un[i] = rt * (s.N / NTW);
      kb[i] = s.K / 128;
      w[i] = i && BF1 != BF ? 2 : 1;
      ks[i] = s.ksplit;
    }
    grid = dec_sk_launch_grid(s1 ? 2 : 1, un, kb, w, ks);
    SLLM_CAPACITY(grid > 0,
                  "stream decode gemm: stream-K ranges cannot keep %d items "
                  "per workgroup", ST_MAX_ITEMS);
    // the kernel deals in 32-bit arithmetic: products of a cost position
    // and a range count stay below 2^31
    const long cmax = un[0] * kb[0] * w[0] + (s1 ? un[1] * kb[1] * w[1] : 0);
    SLLM_REQUIRE(cmax * grid < (1L << 31),
                 "stream decode gemm: stream-K cost line %ld too long for a "
                 "grid of %ld", cmax, grid);
  } else {
    // the kernel deals its items to the XCDs in chunks of (at most) one row
    // tile's items of the first segment (column slabs x K chunks)
    cb = dec_deal_chunk(s0, NTW, upper_items);
    grid = dec_launch_grid(upper_items, cb);
    const long nx = grid / 8;
    const long worst = (chunked_xcd_share(upper_items, cb) + nx - 1) / nx;
    SLLM_CAPACITY(worst <= ST_MAX_ITEMS,
                  "stream decode gemm: %ld items per workgroup above %d "
                  "(upper_items %ld, chunk %ld, grid %ld)", worst,
                  ST_MAX_ITEMS, upper_items, cb, grid);
  }
  SLLM_REQUIRE(grid < (1L << 31), "stream decode gemm: grid too large");
  SegDesc dummy = s0;
  moe_stream_dec_kernel<BF, MODE, true, BM, BF1><<<(unsigned)grid, ST_THREADS, 0, st>>>(
      s0, s1 ? *s1 : dummy, s1 ? 2 : 1, topk, limit, fuse, route, comb,
      (int)cb, sk ? 1 : 0);
  SLLM_LAUNCHED();
  return 0;
}

int launch_stream_dec(int bf, int mode, const SegDesc& s0_in,
                      const SegDesc* s1_in, int topk, float limit,
                      long upper_items, hipStream_t st, int bm,
                      const DecFuse* fuse_in, const RouteInline* route_in,
                      const DecCombine* comb_in, int bf1, bool sk) {
  if (bf1 < 0 || !s1_in) bf1 = bf;
  SLLM_REQUIRE(bf >= 0 && bf <= 2 && (mode == 0 || mode == 1) &&
                   (bm == 16 || bm == 32) &&
                   (bf1 == bf || (bf == SF_FP4 && bf1 != SF_FP4 && bf1 >= 0 &&
                                  bf1 <= 2)),
               "stream decode gemm: bad format (%d, %d) or tile rows %d", bf,
               bf1, bm);
  const int ntw = mode == 0 ? 128 : 256;
  SegDesc seg[2] = {s0_in, s1_in ? *s1_in : s0_in};
  for (int i = 0; i < (s1_in ? 2 : 1); ++i) {
    SegDesc* s = &seg[i];
    if (s->ksplit < 1) s->ksplit = 1;
    SLLM_REQUIRE(s->a && s->wp && s->s0 && s->N % ntw == 0 &&
                     s->K % 128 == 0 && s->K > 0 && s->N / ntw < 32768,
                 "stream decode gemm: bad segment (N=%d K=%d)", s->N, s->K);
    SLLM_REQUIRE(mode == 1 ? s->y != nullptr : s->hq != nullptr,
                 "stream decode gemm: missing outputs");
    SLLM_REQUIRE((i ? bf1 : bf) == SF_FP4 || mode == 1 || s->s1,
                 "stream decode gemm: missing W3 scales");
    SLLM_REQUIRE((!s->gather && !s->row_w_by_idx) || s->sorted_idx,
                 "stream decode gemm: gather / row_w_by_idx need sorted_idx");
    SLLM_REQUIRE(s->tile_info ? s->num_tiles != nullptr : s->total_rows > 0,
                 "stream decode gemm: identity rows need total_rows > 0");
    SLLM_REQUIRE(s->ksplit <= s->K / 128 && s->ksplit < 32768 &&
                     (s->ksplit == 1 ||
                      (s->pstride > 0 && s->pstride % 4 == 0 &&
                       (mode == 1 || (s->pp && !s->row_w)))),
                 "stream decode gemm: bad K split %d (K=%d, mode %d)",
                 s->ksplit, s->K, mode);
  }
  const SegDesc& s0 = seg[0];
  const SegDesc* s1 = s1_in ? &seg[1] : nullptr;
  DecFuse fuse{};
  if (fuse_in && fuse_in->cnt) {
    fuse = *fuse_in;
    SLLM_REQUIRE(mode == 0, "stream decode gemm: only gate/up launches fuse");
    SLLM_REQUIRE(!s1 || fuse.cnt1 > 0, "stream decode gemm: no second counter range");
    for (int i = 0; i < (s1 ? 2 : 1); ++i)
      SLLM_REQUIRE(seg[i].ksplit == 1 ||
                       (seg[i].hq && seg[i].pp && (seg[i].tile_info || i == 1) &&
                        2L * seg[i].ksplit * seg[i].pstride < (1L << 29)),
                   "stream decode gemm: a fused finish needs h, chunk slices "
                   "under 2 GiB, and tile rows for the routed segment");
  }
  RouteInline route{};
  if (route_in && (route_in->logits || route_in->ids_in)) {
    route = *route_in;
    SLLM_REQUIRE(!route.logits || (route.T <= RI_MAX_ROUTE_T && route.ks >= 1 &&
                                   (!route.gate || route.ks > 1) && route.w &&
                                   route.ids && !route.ids_in),
                 "stream decode gemm: bad in-launch routing (T=%d ks=%d)",
                 route.T, route.ks);
    SLLM_REQUIRE(!route.grouped ||
                     (route.logits && route.E <= RI_MAX_E_GROUPED &&
                      route.scoring >= 0 && route.scoring <= 2 &&
                      (route.n_group <= 1 ||
                       (route.n_group <= 64 && route.E % route.n_group == 0 &&
                        route.topk_group >= 1 &&
                        route.topk_group <= route.n_group))),
                 "stream decode gemm: bad in-launch grouped routing (E=%d "
                 "groups %d keep %d)", route.E, route.n_group, route.topk_group);
    SLLM_REQUIRE(mode == 0 && s0.gather && s0.tile_info && s0.sorted_idx &&
                     route.topk == topk && route.bm == bm &&
                     route.max_tiles == s0.max_tiles &&
                     route_inline_fits(route.T, route.E, topk, route.max_tiles) &&
                     route.counts && route.offsets &&
                     route.sorted == s0.sorted_idx && route.inv &&
                     route.tiles == s0.tile_info &&
                     route.ntiles == s0.num_tiles,
                 "stream decode gemm: bad in-launch routing (T=%d E=%d k=%d "
                 "tiles %d)", route.T, route.E, route.topk, route.max_tiles);
    route.nbits = 0;
    while ((1 << route.nbits) < route.E) ++route.nbits;
  }
  DecCombine comb{};
  if (comb_in && comb_in->cnt) {
    comb = *comb_in;
    const long sh_rows = s1 ? s1->total_rows : 0;
    SLLM_REQUIRE(mode == 1 && comb.inv && comb.sorted && comb.out &&
                     comb.y == (const float*)s0.y && comb.ks == s0.ksplit &&
                     comb.kstride == s0.pstride && comb.topk == topk &&
                     comb.topk > 0 && comb.topk <= 64 && comb.H == s0.N &&
                     comb.H % 256 == 0 && s0.tile_info && s0.sorted_idx &&
                     comb.T > 0 && (long)comb.T * comb.topk <= (1L << 24) &&
                     (s1 ? (comb.y_sh == (const float*)s1->y &&
                            comb.ks_sh == s1->ksplit &&
                            comb.kstride_sh == s1->pstride &&
                            sh_rows == comb.T && !s1->tile_info)
                         : comb.y_sh == nullptr) &&
                     4L * comb.ks * comb.kstride < (1L << 31) &&
                     4L * comb.ks_sh * comb.kstride_sh < (1L << 31),
                 "stream decode gemm: bad fused combine (T=%d H=%d k=%d)",
                 comb.T, comb.H, comb.topk);
  }
  // fp32 scale arithmetic covers power-of-two fp8 scales (bf 1)
#define GO(B, M, B1)                                                     \
  return bm == 32 ? go_stream_dec<B, M, 32, B1>(s0, s1, topk, limit, upper_items, st, fuse, route, comb, sk) \
                  : go_stream_dec<B, M, 16, B1>(s0, s1, topk, limit, upper_items, st, fuse, route, comb, sk)
  if (mode == 0) {
    if (bf == SF_FP4 && bf1 != SF_FP4) GO(SF_FP4, 0, SF_FP8_F32S);
    if (bf == SF_FP4) GO(SF_FP4, 0, SF_FP4);
    GO(SF_FP8_F32S, 0, SF_FP8_F32S);
  } else {
    if (bf == SF_FP4 && bf1 != SF_FP4) GO(SF_FP4, 1, SF_FP8_F32S);
    if (bf == SF_FP4) GO(SF_FP4, 1, SF_FP4);
    GO(SF_FP8_F32S, 1, SF_FP8_F32S);
  }
#undef GO
}

long packed_bytes(int fp4, int up, int E, int N, int K) {
  const long NT = up ? N / 128 : N / 256, KB = K / 128;
  return (long)E * NT * KB * (fp4 ? 16384 : 32768);
}

long packed_scale_bytes(int up, int E, int N, int K) {
  const long NT = up ? N / 128 : N / 256, KB = K / 128;
  return (long)E * NT * KB * 1024;
}

}  // namespace sllm

using namespace sllm;

extern "C" {

// 0 when no streamed launch on this device has overflowed its workgroup
// item bound since the last call; otherwise clears the mark and returns -2.
// Synchronizes `stream` first (every launch before the call is covered).
int sllm_moe_stream_status(void* stream) {
  SLLM_HIP(hipStreamSynchronize((hipStream_t)stream));
  int v = 0;
  SLLM_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(stream_item_overflow), sizeof v));
  if (v) {
    const int zero = 0;
    SLLM_HIP(hipMemcpyToSymbol(HIP_SYMBOL(stream_item_overflow), &zero, sizeof zero));
    set_error("a streamed expert GEMM workgroup was dealt more than %d items "
              "and left them undone (host item bound too small)",
              ST_MAX_ITEMS);
    return -2;
  }
  return 0;
}

// Host planning queries (no device work): the ragged tile-count bound and
// the persistent grid the streamed launches use for an item bound.
long sllm_moe_tile_bound(long N, int E, int bm) {
  if (N < 0 || E <= 0 || bm <= 0) {
    set_error("sllm_moe_tile_bound: bad args");
    return -1;
  }
  return tile_bound(N, E, bm);
}

long sllm_moe_stream_grid(long upper_items, int num_cus) {
  if (upper_items < 0 || num_cus <= 0) {
    set_error("sllm_moe_stream_grid: bad args");
    return -1;
  }
  return stream_grid(upper_items, num_cus, ST_MAX_ITEMS);
}

long sllm_moe_stream_dec_grid(long upper_items, int num_cus, long chunk) {
  if (upper_items < 0 || num_cus <= 0 || chunk <= 0) {
    set_error("sllm_moe_stream_dec_grid: bad args");
    return -1;
  }
  return stream_dec_grid(upper_items, num_cus, chunk, ST_MAX_ITEMS);
}

// Size in bytes of the packed weight (and, for fp4, of the packed scales).
long sllm_moe_packed_bytes(int fp4, int up, int E, int N, int K) {
  if (E <= 0 || N <= 0 || K <= 0 || K % 128 || N % (up ? 128 : 256)) {
    set_error("sllm_moe_packed_bytes: need K %% 128 == 0 and N %% %d == 0",
              up ? 128 : 256);
    return -1;
  }
  return packed_bytes(fp4, up, E, N, K);
}

long sllm_moe_packed_scale_bytes(int up, int E, int N, int K) {
  if (E <= 0 || N <= 0 || K <= 0 || K % 128 || N % (up ? 128 : 256)) {
    set_error("sllm_moe_packed_scale_bytes: bad shape");
    return -1;
  }
  return packed_scale_bytes(up, E, N, K);
}

// Repacks expert weights into the streaming layout. fp8: w0 (and w1 for the
// gate/up pair) are (E, N, K) e4m3; fp4: (E, N, K/2) packed e2m1 with e8m0
// scales s0/s1 (E, N, K/32), packed scales to out_scales.
int sllm_moe_pack_weights(int fp4, int up, const void* w0, const void* w1,
                          const void* s0, const void* s1, int E, int N, int K,
                          void* out, void* out_scales, void* stream) {
  SLLM_REQUIRE(w0 && out && (!up || w1), "sllm_moe_pack_weights: null pointer");
  SLLM_REQUIRE(!fp4 || (s0 && out_scales && (!up || s1)),
               "sllm_moe_pack_weights: fp4 needs scales");
  if (sllm_moe_packed_bytes(fp4, up, E, N, K) < 0) return -1;
  const long n = packed_bytes(fp4, up, E, N, K) / 16;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  if (fp4)
    pack_fp4_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
        (const uint8_t*)w0, (const uint8_t*)w1, (const uint8_t*)s0,
        (const uint8_t*)s1, (uint8_t*)out, (uint16_t*)out_scales, E, N, K, up);
  else
    pack_fp8_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
        (const uint8_t*)w0, (const uint8_t*)w1, (uint8_t*)out, E, N, K, up);
  SLLM_LAUNCHED();
  return 0;
}

}  // extern "C"
