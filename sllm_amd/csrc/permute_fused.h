// Single-workgroup pieces of the expert-major permutation, shared by the
// permute launches (permute.hip) and the fused decode route + permute
// kernel (router.hip). Canonical order: ascending expert id, then ascending
// flat assignment index a = t * k + j.
#pragma once
#include "common.h"

namespace sllm {

// Inclusive scan of one int per lane through DPP moves: shifts by 1, 2, 4
// and 8 within each 16-lane row (lanes shifted in from outside the row read
// 0), then row 0's and row 2's last lanes carried into rows 1 and 3, then
// lane 31 into rows 2 and 3.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_shifted(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, 0xF, true);
}

__device__ __forceinline__ int wave_incl_scan(int x) {
  x += dpp_shifted<0x111>(x);  // row_shr:1
  x += dpp_shifted<0x112>(x);  // row_shr:2
  x += dpp_shifted<0x114>(x);  // row_shr:4
  x += dpp_shifted<0x118>(x);  // row_shr:8
  x += dpp_shifted<0x142, 0xA>(x);  // row_bcast:15
  x += dpp_shifted<0x143, 0xC>(x);  // row_bcast:31
  return x;
}

// Block-wide exclusive scan of one value per thread (NW waves, 1024
// threads by default): a DPP scan inside each wave, the NW wave totals
// through LDS, two barriers in all. sh needs NW ints.
template <int NW = 16>
__device__ __forceinline__ int block_excl_scan(int v, int* sh, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int t = sh[w];
    base += w < wave ? t : 0;
    tot += t;
  }
  total = tot;
  __syncthreads();  // sh is reused by the next scan
  return base + x - v;
}

// One workgroup permutes N assignments over E experts: NW waves (1024
// threads in the permutation launches, 512 in the decode gate/up launch
// that routes its own batch), N <= NW G 64, E <= min(HE, NW 64). Wave w
// owns the contiguous assignment range [w R, (w + 1) R) and keeps its ids
// in registers; histogram per wave in LDS, one scan over (expert, wave)
// for counts, offsets, the tile table and each wave's per-expert base,
// then every wave scatters its range in order: lanes holding the same
// expert are matched with one ballot per id bit, so the rank among equal
// ids is the popcount of lower matching lanes (stable, atomic-free). `ids`
// may point to global memory or LDS; hist / sh are the workgroup's LDS
// scratch. The results go to d0 and to d1 (global arrays or LDS copies);
// a null pointer in either is not written.
constexpr int PERM_FUSED_MAX_E = 1024;
constexpr int PERM_FUSED_WAVES = 16;
constexpr int PERM_FUSED_G = 4;  // 64-assignment groups per wave
constexpr int PERM_FUSED_MAX_N = PERM_FUSED_WAVES * PERM_FUSED_G * 64;

struct PermDst {
  int* counts;      // E
  int* offsets;     // E + 1
  int* sorted_idx;  // N
  int* inv_pos;     // N
  int* tile_info;   // 4 max_tiles
  int* num_tiles;   // 1
  // N: the route weight of the assignment at each sorted position (written
  // when the permutation is given the weights by assignment)
  float* rw_sorted = nullptr;
};

template <int NW, int G, int HE>
__device__ __forceinline__ void permute_block(
    const int* ids, int N, int E, int nbits, int bm, int max_tiles,
    const PermDst& d0, const PermDst& d1, int (*hist)[HE], int* sh,
    int* __restrict__ zero = nullptr, int nzero = 0,
    const float* w_src = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < nzero; i += NW * 64) zero[i] = 0;
  const int R = ((N + NW - 1) / NW + 63) & ~63;
  const int a0 = min(N, wave * R), a1 = min(N, a0 + R);
  int idv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int a = a0 + g * 64 + lane;
    const int v = ids[min(a, N - 1)];
    idv[g] = a < a1 ? v : -1;
  }
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < NW; ++w) hist[w][tid] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int e = idv[g];
    if (e >= 0 && e < E) atomicAdd(&hist[wave][e], 1);
  }
  __syncthreads();
  int cnt = 0;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int v = hist[w][tid];
      hist[w][tid] = cnt;
      cnt += v;
    }
  }
  const int ntile = (tid < E && cnt > 0) ? (cnt + bm - 1) / bm : 0;
  int tot_rows, tot_tiles;
  const int off = block_excl_scan<NW>(cnt, sh, tot_rows);
  const int toff = block_excl_scan<NW>(ntile, sh, tot_tiles);
  if (tid < E) {
    if (d0.counts) d0.counts[tid] = cnt;
    if (d1.counts) d1.counts[tid] = cnt;
    if (d0.offsets) d0.offsets[tid] = off;
    if (d1.offsets) d1.offsets[tid] = off;
#pragma unroll
    for (int w = 0; w < NW; ++w) hist[w][tid] += off;
    for (int i = 0; i < ntile && toff + i < max_tiles; ++i) {
      const int r0 = i * bm;
      const int4 t4 = make_int4(tid, off + r0, min(bm, cnt - r0), 0);
      if (d0.tile_info) *(int4*)(d0.tile_info + 4 * (toff + i)) = t4;
      if (d1.tile_info) *(int4*)(d1.tile_info + 4 * (toff + i)) = t4;
    }
  }
  if (tid == 0) {
    if (d0.offsets) d0.offsets[E] = tot_rows;
    if (d1.offsets) d1.offsets[E] = tot_rows;
    if (d0.num_tiles) *d0.num_tiles = min(tot_tiles, max_tiles);
    if (d1.num_tiles) *d1.num_tiles = min(tot_tiles, max_tiles);
  }
  __syncthreads();
  // each wave walks its own range with its own base row: program order
  // within the wave orders the reads and updates of hist[wave][*]
  int* run = hist[wave];
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int a = a0 + g * 64 + lane;
    const int raw = idv[g];
    const bool valid = raw >= 0 && raw < E;
    const int e = valid ? raw : 0;
    if (!valid && a < a1) {  // dropped: the combine skips it
      if (d0.inv_pos) d0.inv_pos[a] = -1;
      if (d1.inv_pos) d1.inv_pos[a] = -1;
    }
    uint64_t peers = __ballot(valid);
    if (peers == 0) continue;  // an empty group (uniform across the wave)
    for (int b = 0; b < nbits; ++b) {
      const int bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int start = valid ? run[e] : 0;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const int pos = start + __popcll(peers & lt);
      if (d0.sorted_idx) d0.sorted_idx[pos] = a;
      if (d1.sorted_idx) d1.sorted_idx[pos] = a;
      if (w_src && d0.rw_sorted) d0.rw_sorted[pos] = w_src[a];
      if (w_src && d1.rw_sorted) d1.rw_sorted[pos] = w_src[a];
      if (d0.inv_pos) d0.inv_pos[a] = pos;
      if (d1.inv_pos) d1.inv_pos[a] = pos;
      if ((peers >> lane) == 1ull) run[e] = start + __popcll(peers);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// The permutation of at most 64 assignments whose experts each hold at most
// bm of them (an expert's rows are one tile: a batch of at most bm tokens
// with distinct experts per token), with permute_block's results. Wave 0
// sorts the keys expert << 6 | assignment with a bitonic network over its
// lanes (dropped assignments, expert outside [0, E), last), so sorted
// position p holds its assignment and each run of one expert is a tile;
// no per-wave histograms over E or block scans. When d0 or d1 takes
// counts / offsets, every thread then finds its experts' runs in the sorted
// keys (keys: 64 words of LDS scratch). The caller synchronizes before
// reading d1.
__device__ __forceinline__ void permute_small_wave(const int* ids, int N, int E,
                                                   int max_tiles,
                                                   const PermDst& d0,
                                                   const PermDst& d1,
                                                   uint32_t* keys,
                                                   const float* w_src = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (wave == 0) {
    const int raw = lane < N ? ids[lane] : -1;
    const bool valid = lane < N && raw >= 0 && raw < E;
    if (lane < N && !valid) {  // dropped: the combine skips it
      if (d0.inv_pos) d0.inv_pos[lane] = -1;
      if (d1.inv_pos) d1.inv_pos[lane] = -1;
    }
    uint32_t key = valid ? ((uint32_t)raw << 6) | (uint32_t)lane : 0xFFFFFFFFu;
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)key, j, kWave);
        const bool keep_min = ((lane & j) == 0) == ((lane & k) == 0);
        key = keep_min ? (o < key ? o : key) : (o > key ? o : key);
      }
    keys[lane] = key;
    const bool v = key != 0xFFFFFFFFu;
    const int e = (int)(key >> 6), a = (int)(key & 63u);
    const int ep = __shfl((int)e, lane > 0 ? lane - 1 : 0, kWave);
    const bool start = v && (lane == 0 || ep != e);
    const uint64_t starts = __ballot(start);
    const int nvalid = __popcll(__ballot(v));
    if (v) {
      if (d0.sorted_idx) d0.sorted_idx[lane] = a;
      if (d1.sorted_idx) d1.sorted_idx[lane] = a;
      if (w_src && d0.rw_sorted) d0.rw_sorted[lane] = w_src[a];
      if (w_src && d1.rw_sorted) d1.rw_sorted[lane] = w_src[a];
      if (d0.inv_pos) d0.inv_pos[a] = lane;
      if (d1.inv_pos) d1.inv_pos[a] = lane;
    }
    if (start) {
      const int t = __popcll(starts & ((1ull << lane) - 1ull));
      const uint64_t later = lane < 63 ? starts >> (lane + 1) : 0ull;
      const int end = later ? lane + 1 + (int)__builtin_ctzll(later) : nvalid;
      if (t < max_tiles) {
        const int4 t4 = make_int4(e, lane, end - lane, 0);
        if (d0.tile_info) *(int4*)(d0.tile_info + 4 * t) = t4;
        if (d1.tile_info) *(int4*)(d1.tile_info + 4 * t) = t4;
      }
    }
    if (lane == 0) {
      const int nt = __popcll(starts) < max_tiles ? __popcll(starts) : max_tiles;
      if (d0.num_tiles) *d0.num_tiles = nt;
      if (d1.num_tiles) *d1.num_tiles = nt;
      if (d0.offsets) d0.offsets[E] = nvalid;
      if (d1.offsets) d1.offsets[E] = nvalid;
    }
  }
  if (d0.counts || d0.offsets || d1.counts || d1.offsets) {
    __syncthreads();  // the sorted keys
    for (int x = tid; x < E; x += blockDim.x) {
      // sorted positions of expert x: [lo, hi), the first keys >= x << 6
      // and >= (x + 1) << 6 (binary searches over the 64 ascending keys)
      int lo = 0, hi = 0;
#pragma unroll
      for (int step = 64; step > 0; step >>= 1) {
        if (lo + step <= 64 && keys[lo + step - 1] < ((uint32_t)x << 6)) lo += step;
        if (hi + step <= 64 && keys[hi + step - 1] < ((uint32_t)(x + 1) << 6))
          hi += step;
      }
      if (d0.counts) d0.counts[x] = hi - lo;
      if (d1.counts) d1.counts[x] = hi - lo;
      if (d0.offsets) d0.offsets[x] = lo;
      if (d1.offsets) d1.offsets[x] = lo;
    }
  }
}

// The permutation launches' form: 16 waves, results to global memory.// The permutation launches' form: 16 waves, results to global memory.
__device__ __forceinline__ void permute_fused_body(
    const int* ids, int N, int E, int nbits, int bm, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ sorted_idx,
    int* __restrict__ inv_pos, int* __restrict__ tile_info,
    int* __restrict__ num_tiles, int max_tiles,
    int (*hist)[PERM_FUSED_MAX_E], int* sh, int* __restrict__ zero = nullptr,
    int nzero = 0) {
  const PermDst d{counts, offsets, sorted_idx, inv_pos, tile_info, num_tiles};
  permute_block<PERM_FUSED_WAVES, PERM_FUSED_G, PERM_FUSED_MAX_E>(
      ids, N, E, nbits, bm, max_tiles, d, PermDst{}, hist, sh, zero, nzero);
}

}  // namespace sllm
