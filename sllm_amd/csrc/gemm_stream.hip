// Persistent, weight-streaming grouped expert GEMMs (prefill) and the packed
// weight layouts they read.
//
// Same arithmetic and epilogues as gemm_grouped.hip (see there for the
// reference semantics); this file changes how the expert weights move:
//
// * Packed weights. A one-time repack (sllm_moe_pack_weights) stores each
//   expert's weights in MFMA operand order: for every (expert, column slab,
//   128-wide K step) one contiguous block holds, wave by wave and subtile by
//   subtile, exactly the bytes each lane feeds the MFMA, so every wave load
//   instruction reads 1 KB of consecutive HBM and a workgroup streams one
//   contiguous 32 KB (fp8) / 16 KB (fp4) block per K step.
// * Persistent workgroups, one per CU (up to 512 registers per lane). Each
//   owns a contiguous run of work items (row tile x column slab, routed
//   items first, then the shared expert's) and walks the flat sequence of
//   (item, K step); the weight operands of step s+2 are in flight while
//   step s computes, across item boundaries, so the weight stream does not
//   drain between tiles. The gathered activation tile of step s+2 is
//   fetched into registers during step s as well and double-buffered in LDS
//   (it comes from L2 / the Infinity Cache, whose latency under this load is
//   microseconds, so one step of lead is not enough).
// * Item descriptors and gathered row indices for the whole run are loaded
//   into LDS once at the start.
#include "launch.h"

namespace sllm {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { SF_FP8_F32S = 0, SF_FP8_POW2 = 1, SF_FP4 = 2 };

constexpr int ST_BM = 128;
constexpr int ST_LDS = 144;          // A row stride in LDS (128 + 16 pad)
constexpr int ST_MAX_ITEMS = 32;     // work items per workgroup

// ---------------------------------------------------------------------------
// packed layouts
// ---------------------------------------------------------------------------
// up   (MODE 0): W1, W3 (E, N, K), N = intermediate, K = hidden; slab = 128
//       h columns, subtile s of wave w = rows 128 nt + 32 w + 16 (s & 1) +
//       (l % 16) of W1 (s < 2) or W3 (s >= 2).
// down (MODE 1): W2 (E, N, K), N = hidden, K = intermediate; slab = 256
//       columns, subtile s of wave w = rows 256 nt + 64 w + 16 s + (l % 16).
// fp8: block (e, nt, kb) = 32 KB at ((e NT + nt) KB + kb) * 32768, inside
//       [w 4][s 4][h 2][lane 64][16 B]: the lane's 32 bytes are K
//       [128 kb + 32 (l / 16), +32), half h = bytes [16 h, 16 h + 16).
// fp4: block = 16 KB, [w][s][lane][16 B]: K [128 kb + 32 (l / 16), +32) =
//       packed bytes [64 kb + 16 (l / 16), +16); e8m0 scales packed as one
//       dword per lane per block: 1 KB blocks [w][lane][s], byte s = scale of
//       (row of subtile s, K block 4 kb + l / 16).
__device__ __forceinline__ int slab_row(int up, int nt, int w, int s, int l) {
  return up ? nt * 128 + w * 32 + (s & 1) * 16 + (l & 15)
            : nt * 256 + w * 64 + s * 16 + (l & 15);
}

__global__ void pack_fp8_kernel(const uint8_t* __restrict__ w0,
                                const uint8_t* __restrict__ w1,
                                uint8_t* __restrict__ out, int E, int N, int K,
                                int up) {
  const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int NT = up ? N / 128 : N / 256, KB = K / 128;
  const long nchunks = (long)E * NT * KB * 2048;
  if (c >= nchunks) return;
  const int l = c & 63, h = (c >> 6) & 1, s = (c >> 7) & 3, w = (c >> 9) & 3;
  const long blk = c >> 11;
  const int kb = (int)(blk % KB);
  const long t = blk / KB;
  const int nt = (int)(t % NT), e = (int)(t / NT);
  const int row = slab_row(up, nt, w, s, l);
  const uint8_t* src = (up && s >= 2) ? w1 : w0;
  const size_t col = (size_t)kb * 128 + (l >> 4) * 32 + h * 16;
  *(uint4*)(out + c * 16) = *(const uint4*)(src + ((size_t)e * N + row) * K + col);
}

__global__ void pack_fp4_kernel(const uint8_t* __restrict__ w0,
                                const uint8_t* __restrict__ w1,
                                const uint8_t* __restrict__ s0,
                                const uint8_t* __restrict__ s1,
                                uint8_t* __restrict__ out,
                                uint32_t* __restrict__ out_s, int E, int N,
                                int K, int up) {
  const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int NT = up ? N / 128 : N / 256, KB = K / 128;
  const long nchunks = (long)E * NT * KB * 1024;
  if (c >= nchunks) return;
  const int l = c & 63, s = (c >> 6) & 3, w = (c >> 8) & 3;
  const long blk = c >> 10;
  const int kb = (int)(blk % KB);
  const long t = blk / KB;
  const int nt = (int)(t % NT), e = (int)(t / NT);
  const int row = slab_row(up, nt, w, s, l);
  const uint8_t* src = (up && s >= 2) ? w1 : w0;
  const size_t col = (size_t)kb * 64 + (l >> 4) * 16;
  *(uint4*)(out + c * 16) =
      *(const uint4*)(src + ((size_t)e * N + row) * (K / 2) + col);
  if (s == 0) {  // one thread per (block, w, lane) writes the scale dword
    uint32_t v = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rq = slab_row(up, nt, w, q, l);
      const uint8_t* sp = (up && q >= 2) ? s1 : s0;
      v |= (uint32_t)sp[((size_t)e * N + rq) * (K / 32) + kb * 4 + (l >> 4)]
           << (8 * q);
    }
    out_s[blk * 256 + w * 64 + l] = v;
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
  v8i v[4];
  uint32_t sc;   // fp4: packed e8m0 scale bytes of the 4 subtiles
  float sb0;     // fp8: W1 / W2 block scale
  float sb1;     // fp8 gate/up: W3 block scale
};

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Streaming (nontemporal) 16-byte load: expert weights are read once per
// layer and should not evict the gathered activation rows from L2.
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  const v4u t = __builtin_nontemporal_load((const v4u*)p);
  return make_uint4(t.x, t.y, t.z, t.w);
}

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

// item descriptor in LDS: x = seg | nt << 1, y = e, z = row_begin, w = rows
template <int BF, int MODE>
__global__ __launch_bounds__(256, 1) void moe_stream_kernel(
    SegDesc S0, SegDesc S1, int nseg, int topk, float limit, int pow2) {
  constexpr int YS = 264;  // bf16 row stride of the down-projection staging
  __shared__ int4 desc[ST_MAX_ITEMS];
  __shared__ int rsrc[ST_MAX_ITEMS][ST_BM];
  __shared__ float rwl[ST_MAX_ITEMS][ST_BM];
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][ST_BM * ST_LDS];
  __shared__ __attribute__((aligned(16))) float sa_lds[2][ST_BM];
  __shared__ __attribute__((aligned(16))) float red[ST_BM][4];
  __shared__ __attribute__((aligned(16))) uint16_t ystage[MODE == 1 ? ST_BM * YS : 8];

  constexpr int NTW = Stream<BF, MODE>::NTW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, lc = lane & 15;

  const int n0 = seg_items<MODE>(S0);
  const int n1 = nseg > 1 ? seg_items<MODE>(S1) : 0;
  const int total = n0 + n1;
  const int chunk = (total + gridDim.x - 1) / gridDim.x;
  const int lo = blockIdx.x * chunk;
  const int hi = min(total, lo + chunk);
  if (lo >= hi || chunk > ST_MAX_ITEMS) return;  // host sizes grid so chunk fits
  const int nitems = hi - lo;

  // ---- phase 0: descriptors and gathered row indices -> LDS ---------------
  if (tid < nitems) {
    const int it = lo + tid;
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
  for (int q = tid; q < nitems * ST_BM; q += 256) {
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

  auto load_b = [&](BSet<BF>& b, int i, int kb) {
    const int4 d = desc[i];
    const int seg = d.x & 1, nt = d.x >> 1;
    const uint8_t* wp = seg ? S1.wp : S0.wp;
    const int N = seg ? S1.N : S0.N, K = seg ? S1.K : S0.K;
    const int NT = N / NTW, KB = K / 128;
    const size_t blk = ((size_t)d.y * NT + nt) * KB + kb;
    const uint8_t* base = wp + blk * Stream<BF, MODE>::BLK;
    if constexpr (BF == SF_FP4) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 v = ld_stream(base + (wave * 4 + s) * 1024 + lane * 16);
        b.v[s] = (v8i){(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
      }
      const uint32_t* sp = (const uint32_t*)(seg ? S1.s0 : S0.s0);
      b.sc = __builtin_nontemporal_load(sp + blk * 256 + wave * 64 + lane);
      b.sb0 = b.sb1 = 0.f;
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 lo4 = ld_stream(base + ((wave * 4 + s) * 2) * 1024 + lane * 16);
        const uint4 hi4 = ld_stream(base + ((wave * 4 + s) * 2 + 1) * 1024 + lane * 16);
        b.v[s] = (v8i){(int)lo4.x, (int)lo4.y, (int)lo4.z, (int)lo4.w,
                       (int)hi4.x, (int)hi4.y, (int)hi4.z, (int)hi4.w};
      }
      b.sc = 0;
      const float* s0p = (const float*)(seg ? S1.s0 : S0.s0);
      if constexpr (MODE == 0) {
        const float* s1p = (const float*)(seg ? S1.s1 : S0.s1);
        const size_t o = ((size_t)d.y * NT + nt) * KB + kb;  // NT = N / 128
        b.sb0 = s0p[o];
        b.sb1 = s1p[o];
      } else {
        const int nblk = (nt * 256 + wave * 64) / 128;
        b.sb0 = b.sb1 = s0p[((size_t)d.y * (N / 128) + nblk) * KB + kb];
      }
    }
  };

  const int my_row = tid >> 1, half = tid & 1;
  struct ASet {
    uint4 v[4];
    float s;
  };
  // Every prefetch load is issued unconditionally (rows past the tile read
  // the valid row 0 of rsrc; they are zeroed when the registers are stored to
  // LDS, after the wait): a load under a branch, which is what the compiler
  // makes of a select applied right after the load, leaves it no guaranteed
  // count of younger loads and forces a wait that drains the pipeline.
  // Thread tid gathers 16-byte chunk (tid & 7) of tile rows 32 q + tid / 8:
  // each load instruction of a wave reads eight whole 128-byte row segments.
  const int a_chunk = tid & 7, a_row0 = tid >> 3;
  auto fetch_a = [&](ASet& af, int i, int kb) {
    const int4 d = desc[i];
    const SegDesc& S = (d.x & 1) ? S1 : S0;
    const int K = S.K, KB = K / 128;
    const uint8_t* base = S.a + kb * 128 + a_chunk * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      af.v[q] = *(const uint4*)(base + (size_t)rsrc[i][q * 32 + a_row0] * K);
    af.s = S.sa[(size_t)rsrc[i][tid & (ST_BM - 1)] * KB + kb];
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[mi][s] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // cursors: compute (ci, ckb), B prefetch (bi, bkb), A prefetch (ai, akb)
  int ci = 0, ckb = 0, bi = 0, bkb = 0, ai = 0, akb = 0;
  auto adv = [&](int& i, int& kb) {
    if (++kb == kb_of(i)) {
      kb = 0;
      ++i;
    }
  };
  // prefetch cursors saturate at the last step (the surplus loads at the end
  // of the run re-read the last block and are never consumed)
  auto adv_sat = [&](int& i, int& kb) {
    if (kb + 1 < kb_of(i)) {
      ++kb;
    } else if (i + 1 < nitems) {
      kb = 0;
      ++i;
    }
  };

  // ---- epilogues ------------------------------------------------------------
  // acc[mi][s][v] holds token mi * 16 + lc (tile row) and output column
  // 16 s + 4 lg + v of the wave's subtiles.
  auto epilogue = [&](int i, int ebuf) {
    const int4 d = desc[i];
    const int seg = d.x & 1, nt = d.x >> 1;
    const SegDesc& S = seg ? S1 : S0;
    const int rows = d.w, rb = d.z;
    const int nmi = (rows + 15) >> 4;
    if constexpr (MODE == 0) {
      // h = silu(g) * u * route weight over the wave's 32 columns (gate
      // subtiles 0, 1; up subtiles 2, 3), row amax across lane groups and
      // then across the four waves, requantised per row to e4m3.
      const int ntn = S.N / 128;
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        if (mi < nmi) {
          const int t = mi * 16 + lc;
          const float rw = rwl[i][t];
          float amax = 0.f;
#pragma unroll
          for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              float g = acc[mi][s][v], u = acc[mi][s + 2][v];
              if (limit > 0.f) {
                u = fminf(fmaxf(u, -limit), limit);
                g = fminf(g, limit);
              }
              const float h = silu_fast(g) * u * rw;
              acc[mi][s][v] = h;
              amax = fmaxf(amax, fabsf(h));
            }
          }
          amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
          amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
          if (lg == 0) red[t][wave] = amax;
        }
      }
      __syncthreads();
      uint8_t* h_lds = a_lds[ebuf];
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        if (mi < nmi) {
          const int t = mi * 16 + lc;
          const float4 r4 = *(const float4*)red[t];
          const float amax = fmaxf(fmaxf(r4.x, r4.y), fmaxf(r4.z, r4.w));
          float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
          if (pow2) {
            const uint32_t bits = __float_as_uint(sc);
            const int ex = (int)((bits >> 23) & 0xFF) - 127 +
                           ((bits & 0x7FFFFF) ? 1 : 0);
            sc = __uint_as_float((uint32_t)(ex + 127) << 23);
          }
          const float inv = 1.0f / sc;
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            float y[4];
#pragma unroll
            for (int v = 0; v < 4; ++v)
              y[v] = fminf(fmaxf(acc[mi][s][v] * inv, -448.f), 448.f);
            *(uint32_t*)(h_lds + t * ST_LDS + wave * 32 + s * 16 + lg * 4) =
                f32x4_to_e4m3(y[0], y[1], y[2], y[3]);
          }
          if (wave == 0 && lg == 0 && t < rows)
            S.hs[(size_t)(rb + t) * ntn + nt] = sc;
        }
      }
      __syncthreads();
      if (my_row < rows) {
        const uint4* p = (const uint4*)(h_lds + my_row * ST_LDS + half * 64);
        uint4* dst = (uint4*)(S.hq + (size_t)(rb + my_row) * S.N + nt * 128 + half * 64);
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[q] = p[q];
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
          for (int s = 0; s < 4; ++s) {
            const uint32_t lo = (uint32_t)f32_to_bf16(acc[mi][s][0] * w) |
                                ((uint32_t)f32_to_bf16(acc[mi][s][1] * w) << 16);
            const uint32_t hi = (uint32_t)f32_to_bf16(acc[mi][s][2] * w) |
                                ((uint32_t)f32_to_bf16(acc[mi][s][3] * w) << 16);
            *(uint2*)(ystage + t * YS + wave * 64 + s * 16 + lg * 4) =
                make_uint2(lo, hi);
          }
        }
      }
      __syncthreads();
      for (int c = tid; c < rows * 32; c += 256) {
        const int r = c >> 5, c8 = c & 31;
        *(uint4*)(S.y + (size_t)(rb + r) * S.N + nt * 256 + c8 * 8) =
            *(const uint4*)(ystage + r * YS + c8 * 8);
      }
      __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[mi][s] = (f32x4){0.f, 0.f, 0.f, 0.f};
  };

  // ---- one pipeline step ----------------------------------------------------
  auto step = [&](int st, ASet& acur, ASet& aload, BSet<BF>& bcur,
                  BSet<BF>& bload) {
    const int buf = st & 1;
    const int4 d = desc[ci];
    {  // A(st) registers -> LDS, rows past the tile zeroed
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = q * 32 + a_row0;
        const uint32_t m = r < d.w ? ~0u : 0u;
        const uint4 v = acur.v[q];
        *(uint4*)(a_lds[buf] + r * ST_LDS + a_chunk * 16) =
            make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
      }
      const uint32_t ms = tid < d.w ? ~0u : 0u;
      if (tid < ST_BM) sa_lds[buf][tid] = __uint_as_float(__float_as_uint(acur.s) & ms);
    }
    __syncthreads();
    // both operands are prefetched three steps ahead; the activations of a
    // step are consumed before its weights, so they are issued first
    fetch_a(aload, ai, akb);
    adv_sat(ai, akb);
    load_b(bload, bi, bkb);
    adv_sat(bi, bkb);
    // compute step st over all eight 16-row groups: rows past the tile are
    // zero in LDS, and a branch-free step lets the compiler issue the LDS
    // reads of the next groups ahead of the MFMAs of the current one.
    const int seg = d.x & 1;
    const SegDesc& S = seg ? S1 : S0;
    const int KB = S.K / 128;
    const uint8_t* lds = a_lds[buf];
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
      // lane's four values share one token, so one scale product per
      // subtile pair. The MFMAs of row group mi run while the partials of
      // group mi - 1 are rescaled, from a second set of partial registers.
      const float sb0 = bcur.sb0, sb1 = MODE == 0 ? bcur.sb1 : bcur.sb0;
      f32x4 part[2][4];
      auto rescale = [&](int m) {
        const float sx = sa_lds[buf][m * 16 + lc];
        const float f0 = sx * sb0, f1 = sx * sb1;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float f = s < 2 ? f0 : f1;
#pragma unroll
          for (int v = 0; v < 4; ++v)
            acc[m][s][v] = fmaf(part[m & 1][s][v], f, acc[m][s][v]);
        }
      };
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        const v8i x = a_frag(mi);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          part[mi & 1][s] = st_mma<BF>(bcur.v[s], x, part[mi & 1][s], 0, 0);
        if (mi > 0) rescale(mi - 1);
      }
      rescale(7);
    } else {
      const float sbf[2] = {bcur.sb0, bcur.sb1};
      uint32_t sbe[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sbe[s] = BF == SF_FP4 ? (bcur.sc >> (8 * s)) & 0xFF
                              : e8m0_bits(sbf[MODE == 0 ? (s >> 1) : 0]);
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        const v8i x = a_frag(mi);
        const uint32_t sxe = e8m0_bits(sa_lds[buf][mi * 16 + lc]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          acc[mi][s] = st_mma<BF>(bcur.v[s], x, acc[mi][s], sbe[s], sxe);
      }
    }
    const bool last = ckb + 1 == KB;
    const int cur_item = ci;
    adv(ci, ckb);
    if (last) epilogue(cur_item, buf ^ 1);
  };

  // ---- pipeline -------------------------------------------------------------
  // Four register sets per operand, prefetch distance 3. The loop body runs
  // its four steps unconditionally: a conditional step would make the
  // compiler's wait analysis at the back-edge merge a path whose most recent
  // loads are older, and wait for everything.
  BSet<BF> b0, b1, b2, b3;
  ASet a0, a1, a2, a3;
  fetch_a(a0, ai, akb);
  adv_sat(ai, akb);
  load_b(b0, bi, bkb);
  adv_sat(bi, bkb);
  fetch_a(a1, ai, akb);
  adv_sat(ai, akb);
  load_b(b1, bi, bkb);
  adv_sat(bi, bkb);
  fetch_a(a2, ai, akb);
  adv_sat(ai, akb);
  load_b(b2, bi, bkb);
  adv_sat(bi, bkb);
  int st = 0;
  for (; st + 4 <= total_steps; st += 4) {
    step(st, a0, a3, b0, b3);
    step(st + 1, a1, a0, b1, b0);
    step(st + 2, a2, a1, b2, b1);
    step(st + 3, a3, a2, b3, b2);
  }
  if (st < total_steps) step(st, a0, a3, b0, b3);
  if (st + 1 < total_steps) step(st + 1, a1, a0, b1, b0);
  if (st + 2 < total_steps) step(st + 2, a2, a1, b2, b1);
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

// upper_items: an upper bound of the total item count (sizes the grid so
// that no workgroup receives more than ST_MAX_ITEMS items).
template <int BF, int MODE>
static int go_stream(const SegDesc& s0, const SegDesc* s1, int topk,
                     float limit, int pow2, long upper_items, hipStream_t st) {
  const long need = (upper_items + ST_MAX_ITEMS - 1) / ST_MAX_ITEMS;
  const long grid = need > num_cus() ? need : num_cus();
  SLLM_REQUIRE(grid < (1L << 31), "stream gemm: grid too large");
  SegDesc dummy = s0;
  moe_stream_kernel<BF, MODE><<<(unsigned)grid, 256, 0, st>>>(
      s0, s1 ? *s1 : dummy, s1 ? 2 : 1, topk, limit, pow2);
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
        (const uint8_t*)s1, (uint8_t*)out, (uint32_t*)out_scales, E, N, K, up);
  else
    pack_fp8_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
        (const uint8_t*)w0, (const uint8_t*)w1, (uint8_t*)out, E, N, K, up);
  SLLM_LAUNCHED();
  return 0;
}

}  // extern "C"
