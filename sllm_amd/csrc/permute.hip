// Expert-major token permutation (dispatch) and the ragged tile table.
//
// The reference has no permute: its numpy oracle loops per token
// (ref/qwen4_exp.py:175-179) or per expert with np.where
// (ref/deepseek_v4.py:1080-1086, upstream ref/hf_sources/dsv4/model.py:
// 689-695 torch.where(indices == i)). This file produces the same
// grouping as an explicit permutation so that each expert's rows are
// contiguous for the grouped GEMMs.
//
// Canonical order (bit-exact with oracle/permute.py): ascending expert id,
// then ascending flat assignment index a = t*k + j, i.e.
// np.argsort(ids.ravel(), kind="stable").
//
// Small problems use one fused workgroup (permute_fused_kernel); up to 1024
// experts, hist followed by permute_chunk_kernel (scan and scatter in one
// launch); otherwise three kernels, all deterministic:
//  1. hist:    chunks of PERM_CHUNK assignments, LDS histogram per chunk.
//  2. scan:    one workgroup; per-expert exclusive scan over chunks, then an
//              exclusive scan over experts (offsets), chunk bases, and the
//              tile table: ceil(count/bm) tiles per expert, each an int4
//              {expert, first permuted row, rows, 0}.
//  3. scatter: one wave per chunk walks its assignments in order, 64 at a
//              time; lanes holding the same expert are matched with one
//              ballot per id bit, so the rank among equal ids is the popcount
//              of lower matching lanes -- a stable, atomic-free scatter.
#include "launch.h"
#include "permute_fused.h"

namespace sllm {

constexpr int PERM_SCAN_REG = 48;  // chunk counts an expert keeps in registers

__global__ __launch_bounds__(256) void permute_hist_kernel(
    const int* __restrict__ ids, int N, int E, int* __restrict__ chunk_hist) {
  extern __shared__ int h[];
  const int c = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += blockDim.x) h[e] = 0;
  __syncthreads();
  const int a0 = c * PERM_CHUNK, a1 = min(N, a0 + PERM_CHUNK);
  for (int a = a0 + threadIdx.x; a < a1; a += blockDim.x) {
    int e = ids[a];
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    chunk_hist[(size_t)c * E + e] = h[e];
}

__global__ __launch_bounds__(1024) void permute_scan_kernel(
    int* __restrict__ chunk_hist, int nchunks, int E, int bm,
    int* __restrict__ counts, int* __restrict__ offsets,
    int* __restrict__ tile_info, int* __restrict__ num_tiles, int max_tiles) {
  __shared__ int sh[1024];
  __shared__ int carry_rows, carry_tiles;
  const int tid = threadIdx.x;
  if (tid == 0) {
    carry_rows = 0;
    carry_tiles = 0;
  }
  __syncthreads();
  for (int e0 = 0; e0 < E; e0 += 1024) {
    const int e = e0 + tid;
    // The expert's chunk counts stay in registers between the count and
    // the base pass (chunks beyond PERM_SCAN_REG are re-read). All loads of
    // a batch are in flight at once: a dependent load per chunk would expose
    // the memory latency nchunks times.
    int v[PERM_SCAN_REG];
    int cnt = 0;
    if (e < E) {
#pragma unroll
      for (int j = 0; j < PERM_SCAN_REG; ++j)
        v[j] = j < nchunks ? chunk_hist[(size_t)j * E + e] : 0;
#pragma unroll
      for (int j = 0; j < PERM_SCAN_REG; ++j) cnt += v[j];
      for (int c0 = PERM_SCAN_REG; c0 < nchunks; c0 += 8) {
        int w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          w[j] = c0 + j < nchunks ? chunk_hist[(size_t)(c0 + j) * E + e] : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) cnt += w[j];
      }
    }
    int ntile = (e < E && cnt > 0) ? (cnt + bm - 1) / bm : 0;
    int tot_rows, tot_tiles;
    int off = block_excl_scan(cnt, sh, tot_rows) + carry_rows;
    int toff = block_excl_scan(ntile, sh, tot_tiles) + carry_tiles;
    if (e < E) {
      counts[e] = cnt;
      offsets[e] = off;
      // chunk bases: the expert's offset plus its exclusive prefix over
      // chunks
      int run = off;
#pragma unroll
      for (int j = 0; j < PERM_SCAN_REG; ++j) {
        if (j < nchunks) chunk_hist[(size_t)j * E + e] = run;
        run += v[j];
      }
      for (int c0 = PERM_SCAN_REG; c0 < nchunks; c0 += 8) {
        int w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          w[j] = c0 + j < nchunks ? chunk_hist[(size_t)(c0 + j) * E + e] : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (c0 + j < nchunks) chunk_hist[(size_t)(c0 + j) * E + e] = run;
          run += w[j];
        }
      }
      for (int i = 0; i < ntile && toff + i < max_tiles; ++i) {
        const int r0 = i * bm;
        *(int4*)(tile_info + 4 * (toff + i)) =
            make_int4(e, off + r0, min(bm, cnt - r0), 0);
      }
    }
    __syncthreads();
    if (tid == 0) {
      carry_rows += tot_rows;
      carry_tiles += tot_tiles;
    }
    __syncthreads();
  }
  if (tid == 0) {
    offsets[E] = carry_rows;
    *num_tiles = min(carry_tiles, max_tiles);
  }
}

__global__ __launch_bounds__(64) void permute_scatter_kernel(
    const int* __restrict__ ids, int N, int E, int nbits,
    const int* __restrict__ chunk_base, int* __restrict__ sorted_idx,
    int* __restrict__ inv_pos) {
  extern __shared__ int run[];
  const int c = blockIdx.x;
  const int lane = threadIdx.x;
  // the chunk's expert bases, eight loads in flight per lane
  for (int e0 = 0; e0 < E; e0 += 512) {
    int b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = e0 + j * 64 + lane;
      b[j] = e < E ? chunk_base[(size_t)c * E + e] : 0;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = e0 + j * 64 + lane;
      if (e < E) run[e] = b[j];
    }
  }
  __syncthreads();
  const int a0 = c * PERM_CHUNK, a1 = min(N, a0 + PERM_CHUNK);
  const uint64_t lt = (1ull << lane) - 1ull;
  // the chunk's ids, all loads in flight at once (clamped in-bounds)
  constexpr int G = PERM_CHUNK / 64;
  int idv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) idv[g] = ids[min(a0 + g * 64 + lane, N - 1)];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int base = a0 + g * 64;
    if (base >= a1) break;
    const int a = base + lane;
    const int raw = a < a1 ? idv[g] : -1;
    const bool valid = raw >= 0 && raw < E;  // out-of-range ids are dropped
    const int e = valid ? raw : 0;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const int bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    if (valid) {
      const int rank = __popcll(peers & lt);
      const int pos = run[e] + rank;
      sorted_idx[pos] = a;
      inv_pos[a] = pos;
    } else if (a < a1) {
      inv_pos[a] = -1;  // a dropped assignment: the combine skips it
    }
    __syncthreads();  // every lane has read run[] before it advances
    if (valid && (peers >> lane) == 1ull) run[e] += __popcll(peers);
    __syncthreads();
  }
}

// Scan and scatter in one launch (E <= PERM_FUSED_MAX_E): workgroup c owns
// chunk c (16 waves x 64 assignments) and derives everything it needs from
// the chunk histograms itself -- every expert's total (an exclusive scan of
// the totals gives the expert offsets) and the expert's count in earlier
// chunks -- so no single-workgroup scan pass runs in between. Within the
// chunk, per-wave LDS histograms give each wave its per-expert base, and
// the waves scatter their 64 assignments with ballot ranks. Workgroup 0 also
// writes counts, offsets and the tile table.
__global__ __launch_bounds__(1024) void permute_chunk_kernel(
    const int* __restrict__ ids, int N, int E, int nbits, int bm, int nchunks,
    const int* __restrict__ chunk_hist, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ sorted_idx,
    int* __restrict__ inv_pos, int* __restrict__ tile_info,
    int* __restrict__ num_tiles, int max_tiles) {
  __shared__ int hist[PERM_FUSED_WAVES][PERM_FUSED_MAX_E];
  __shared__ int sh[1024];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x;
  const int a = c * PERM_CHUNK + wave * 64 + lane;
  const int raw = a < N ? ids[a] : -1;
  for (int q = tid; q < PERM_FUSED_WAVES * E; q += 1024) hist[q / E][q % E] = 0;
  // expert tid: total over all chunks and count in the chunks before c
  int tot = 0, pre = 0;
  if (tid < E) {
    for (int c0 = 0; c0 < nchunks; c0 += 16) {
      int v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        v[j] = c0 + j < nchunks ? chunk_hist[(size_t)(c0 + j) * E + tid] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        tot += v[j];
        pre += c0 + j < c ? v[j] : 0;
      }
    }
  }
  __syncthreads();
  const bool valid = raw >= 0 && raw < E;  // out-of-range ids are dropped
  if (valid) atomicAdd(&hist[wave][raw], 1);
  int tot_rows, tot_tiles;
  const int off = block_excl_scan(tot, sh, tot_rows);  // (its barriers also
                                                       // order the atomics)
  if (c == 0) {
    const int ntile = (tid < E && tot > 0) ? (tot + bm - 1) / bm : 0;
    const int toff = block_excl_scan(ntile, sh, tot_tiles);
    if (tid < E) {
      counts[tid] = tot;
      offsets[tid] = off;
      for (int i = 0; i < ntile && toff + i < max_tiles; ++i) {
        const int r0 = i * bm;
        *(int4*)(tile_info + 4 * (toff + i)) =
            make_int4(tid, off + r0, min(bm, tot - r0), 0);
      }
    }
    if (tid == 0) {
      offsets[E] = tot_rows;
      *num_tiles = min(tot_tiles, max_tiles);
    }
  }
  if (tid < E) {  // per-wave bases of expert tid within the chunk
    int run = off + pre;
#pragma unroll
    for (int w = 0; w < PERM_FUSED_WAVES; ++w) {
      const int h = hist[w][tid];
      hist[w][tid] = run;
      run += h;
    }
  }
  __syncthreads();
  const int e = valid ? raw : 0;
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const int bit = (e >> b) & 1;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  if (valid) {
    const int pos = hist[wave][e] + __popcll(peers & ((1ull << lane) - 1ull));
    sorted_idx[pos] = a;
    inv_pos[a] = pos;
  } else if (a < N) {
    inv_pos[a] = -1;  // a dropped assignment: the combine skips it
  }
}

__global__ __launch_bounds__(1024) void permute_fused_kernel(
    const int* __restrict__ ids, int N, int E, int nbits, int bm,
    int* __restrict__ counts, int* __restrict__ offsets,
    int* __restrict__ sorted_idx, int* __restrict__ inv_pos,
    int* __restrict__ tile_info, int* __restrict__ num_tiles, int max_tiles,
    int* __restrict__ zero, int nzero) {
  __shared__ int hist[PERM_FUSED_WAVES][PERM_FUSED_MAX_E];
  __shared__ int sh[1024];
  permute_fused_body(ids, N, E, nbits, bm, counts, offsets, sorted_idx,
                     inv_pos, tile_info, num_tiles, max_tiles, hist, sh, zero,
                     nzero);
}

bool permute_uses_chunk_hist(int N, int E) {
  return !(N <= PERM_FUSED_MAX_N && E <= PERM_FUSED_MAX_E);
}

size_t permute_scratch_bytes(int N, int E) {
  int nchunks = N > 0 ? (N + PERM_CHUNK - 1) / PERM_CHUNK : 1;
  return align_up((size_t)nchunks * E * sizeof(int), 256);
}

// ids (N = T*k) int32 -> counts[E], offsets[E+1], sorted_idx[N], inv_pos[N],
// tile_info[4*max_tiles] {expert, first row, rows, 0}, num_tiles[1].
int launch_permute(const int* ids, int N, int E, int bm, int* counts,
                   int* offsets, int* sorted_idx, int* inv_pos,
                   int* tile_info, int* num_tiles, int max_tiles,
                   void* scratch, hipStream_t st, bool hist_ready,
                   int* zero, int nzero) {
  SLLM_REQUIRE(ids && counts && offsets && sorted_idx && inv_pos &&
                   tile_info && num_tiles && scratch,
               "permute: null pointer");
  SLLM_REQUIRE(nzero == 0 || (zero && nzero > 0 && !permute_uses_chunk_hist(N, E)),
               "permute: zeroing needs the one-workgroup permutation");
  SLLM_REQUIRE(N > 0 && E > 0 && E <= 4096 && bm > 0,
               "permute: bad sizes (N=%d E=%d bm=%d)", N, E, bm);
  const int nchunks = (N + PERM_CHUNK - 1) / PERM_CHUNK;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  if (!permute_uses_chunk_hist(N, E)) {
    permute_fused_kernel<<<1, 1024, 0, st>>>(ids, N, E, nbits, bm, counts,
                                             offsets, sorted_idx, inv_pos,
                                             tile_info, num_tiles, max_tiles,
                                             zero, nzero);
    SLLM_LAUNCHED();
    return 0;
  }
  int* chunk_hist = (int*)scratch;
  const size_t lds = (size_t)E * sizeof(int);
  if (!hist_ready) {  // else filled by the routing launch
    permute_hist_kernel<<<nchunks, 256, lds, st>>>(ids, N, E, chunk_hist);
    SLLM_LAUNCHED();
  }
  if (E <= PERM_FUSED_MAX_E) {
    static_assert(PERM_CHUNK == PERM_FUSED_WAVES * 64, "one group per wave");
    permute_chunk_kernel<<<nchunks, 1024, 0, st>>>(
        ids, N, E, nbits, bm, nchunks, chunk_hist, counts, offsets, sorted_idx,
        inv_pos, tile_info, num_tiles, max_tiles);
    SLLM_LAUNCHED();
    return 0;
  }
  permute_scan_kernel<<<1, 1024, 0, st>>>(chunk_hist, nchunks, E, bm, counts,
                                          offsets, tile_info, num_tiles,
                                          max_tiles);
  SLLM_LAUNCHED();
  permute_scatter_kernel<<<nchunks, 64, lds, st>>>(
      ids, N, E, nbits, chunk_hist, sorted_idx, inv_pos);
  SLLM_LAUNCHED();
  return 0;
}

}  // namespace sllm

using namespace sllm;

extern "C" {

long sllm_moe_permute_scratch_bytes(int N, int E) {
  return (long)permute_scratch_bytes(N, E);
}

int sllm_moe_permute(const int* ids, int N, int E, int bm, int* counts,
                     int* offsets, int* sorted_idx, int* inv_pos,
                     int* tile_info, int* num_tiles, int max_tiles,
                     void* scratch, void* stream) {
  return launch_permute(ids, N, E, bm, counts, offsets, sorted_idx, inv_pos,
                        tile_info, num_tiles, max_tiles, scratch,
                        (hipStream_t)stream);
}

}  // extern "C"
