// Per-token routing on one wave, shared by the routing launches
// (router.hip) and the decode gate/up launch that routes its batch itself
// (gemm_stream.hip): top-k keys, the wave's top-k, the logits of a row held
// as K-chunk slices, the softmax weights (ref/qwen4_exp.py:118-140; tie
// rule of kernels/cuda/qwen4.cu:259-270), and the scored, biased and
// group-limited routing (ref/deepseek_v4.py:522-561).
#pragma once
#include "common.h"

namespace sllm {

// --------------------------------------------------------------------------
// softmax top-k with renormalisation (ref/qwen4_exp.py:118-140)
// --------------------------------------------------------------------------
// Top-k keys: the order key of the value (f32_order_key) in the high half,
// ~e in the low half, so that a larger key is a larger value and, among
// equal values, the lower expert id e; 0 = no candidate. -0 is keyed as +0:
// the two are equal values (and give equal probabilities), so they tie.
__device__ __forceinline__ uint64_t topk_key(float v, int e) {
  v = v == 0.f ? 0.f : v;
  return ((uint64_t)f32_order_key(v) << 32) |
         (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}

__device__ __forceinline__ float topk_key_value(uint64_t key) {
  const uint32_t k = (uint32_t)(key >> 32);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ int topk_key_id(uint64_t key) {
  return (int)(0xFFFFFFFFu - (uint32_t)key);
}

// Descending sorting networks (2, 4, 8 inputs: 1, 5, 19 comparators).
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&k)[N]) {
  auto ce = [&](int i, int j) {
    const uint64_t a = k[i], b = k[j];
    const bool sw = b > a;
    k[i] = sw ? b : a;
    k[j] = sw ? a : b;
  };
  if constexpr (N == 2) {
    ce(0, 1);
  } else if constexpr (N == 4) {
    ce(0, 1); ce(2, 3); ce(0, 2); ce(1, 3); ce(1, 2);
  } else if constexpr (N == 8) {
    ce(0, 2); ce(1, 3); ce(4, 6); ce(5, 7);
    ce(0, 4); ce(1, 5); ce(2, 6); ce(3, 7);
    ce(0, 1); ce(2, 3); ce(4, 5); ce(6, 7);
    ce(2, 4); ce(3, 5);
    ce(1, 4); ce(3, 6);
    ce(1, 2); ce(3, 4); ce(5, 6);
  }
}

// Descending top-k of the wave's candidate keys (key[i] of each lane, 0 =
// none; keys are distinct, as each carries its expert id); lane j < topk
// returns pick j's key (0 past the candidates).
// Up to 8 keys per lane: each lane sorts its keys once, then every pick
// is one wave maximum of the lanes' heads and a pop on the owning lane.
// More keys per lane: every pick takes the lane maxima afresh.
template <int EPL>
__device__ __forceinline__ uint64_t wave_topk_keys(uint64_t (&key)[EPL],
                                                   int topk) {
  const int lane = threadIdx.x & 63;
  uint64_t mine = 0;
  if constexpr (EPL <= 8) {
    sort_desc<EPL>(key);
    for (int kk = 0; kk < topk; ++kk) {
      // the maximum of the value halves; the full 64-bit keys only decide
      // between lanes that share it
      const uint32_t hi = (uint32_t)(key[0] >> 32);
      const uint32_t mhi = wave_max_u32(hi);
      const uint64_t bal = __ballot(hi == mhi);
      uint64_t best;
      if (__popcll(bal) == 1) {
        const int owner = (int)__builtin_ctzll(bal);
        best = ((uint64_t)mhi << 32) |
               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], owner);
      } else {
        best = wave_max_u64(hi == mhi ? key[0] : 0ull);
      }
      if (lane == kk) mine = best;
      if (best != 0 && key[0] == best) {  // the one lane whose head it is
#pragma unroll
        for (int i = 0; i + 1 < EPL; ++i) key[i] = key[i + 1];
        key[EPL - 1] = 0;
      }
    }
  } else {
    for (int kk = 0; kk < topk; ++kk) {
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < EPL; ++i) best = key[i] > best ? key[i] : best;
      best = wave_max_u64(best);
      if (lane == kk) mine = best;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (best != 0 && key[i] == best) key[i] = 0;
    }
  }
  return mine;
}

// The calling wave's logits of one row (lane holds experts lane + 64 i;
// fill past E) when the row is held as ks K-chunk slices kstride floats
// apart (the split decode router GEMM): slices are added in order, the
// loads of G slices in flight together. With several slices
// the owning wave (store) writes the sums back into slice 0, which then
// holds the logits the routing used (the debug copy reads slice 0).
// G: slices whose loads are in flight together (registers: G * EPL).
template <int EPL, int G = (EPL >= 64 ? 1 : (64 / EPL < 8 ? 64 / EPL : 8))>
__device__ __forceinline__ void logit_sums(float* row, int ks, long kstride,
                                           int E, bool store, float fill,
                                           float (&v)[EPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? row[e] : fill;
  }
  if (ks <= 1) return;
  for (int q0 = 1; q0 < ks; q0 += G) {
    float t[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int e = lane + 64 * i;
        t[g][i] = q0 + g < ks && e < E ? row[(q0 + g) * kstride + e] : 0.f;
      }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < EPL; ++i) v[i] += t[g][i];
  }
  if (store) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      if (e < E) row[e] = v[i];
    }
  }
}

// Lane j < topk holds pick j; m and s are the row's largest logit and sum
// of exp(l - m): pick j's probability is exp(l - m) / s, and the weights
// are those probabilities over their sum in pick order plus eps
// (ref/qwen4_exp.py:118-140). A null w_row writes slot j to id_lds only
// (then id_row is not written either).
__device__ __forceinline__ void softmax_emit(uint64_t pick, float m, float s,
                                             int topk, float eps,
                                             float* __restrict__ w_row,
                                             int* __restrict__ id_row,
                                             int* id_lds,
                                             float* w_lds = nullptr) {
  const int lane = threadIdx.x & 63;
  const float pn = expf(topk_key_value(pick) - m) / s;  // lane j: pick j
  float wsum = 0.f;
  for (int j = 0; j < topk; ++j)
    wsum += __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(pn), j));
  if (lane < topk) {
    const int myid = topk_key_id(pick);
    if (w_row) {
      w_row[lane] = pn / (wsum + eps);
      id_row[lane] = myid;
    }
    if (id_lds) id_lds[lane] = myid;
    if (w_lds) w_lds[lane] = pn / (wsum + eps);
  }
}

// One token's softmax top-k on the calling wave: row = the token's E logits
// (plus bias[e] when bias is given, after the slices are added; the row
// keeps the logits without it); lanes j < topk write slot j of w_row /
// id_row (and of id_lds when given). store: with several slices, write
// the logits (their sum) back into slice 0 (logit_sums); a caller whose
// row other workgroups read at the same time passes false.
// The selection runs on the logits (softmax is monotone in them); pick j's
// probability is exp(l - max) / sum recomputed from its key, and the
// weights are those probabilities over their sum in pick order plus eps
// (ref/qwen4_exp.py:118-140).
template <int EPL, int G = (EPL >= 64 ? 1 : (64 / EPL < 8 ? 64 / EPL : 8))>
__device__ __forceinline__ void route_softmax_token(
    float* row, int ks, long kstride, int E, int topk, float eps,
    float* __restrict__ w_row, int* __restrict__ id_row, int* id_lds,
    const float* __restrict__ bias, bool store = true,
    float* w_lds = nullptr) {
  const int lane = threadIdx.x & 63;
  float v[EPL];
  logit_sums<EPL, G>(row, ks, kstride, E, store, -INFINITY, v);
  if (bias) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      if (e < E) v[i] += bias[e];
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) m = fmaxf(m, v[i]);
  m = wave_max(m);
  float s = 0.f;
  uint64_t key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = lane + 64 * i;
    s += e < E ? expf(v[i] - m) : 0.f;
    key[i] = e < E ? topk_key(v[i], e) : 0ull;
  }
  s = wave_sum(s);
  const uint64_t pick = wave_topk_keys<EPL>(key, topk);
  softmax_emit(pick, m, s, topk, eps, w_row, id_row, id_lds, w_lds);
}

// Token t's shared-expert gate from the split router GEMM's ks partial
// logits (gate[T + q T + t]): added in chunk order, sigmoid into gate[t].
__device__ __forceinline__ void route_gate_finish(float* gate, int T, int t,
                                                  int ks) {
  float g = gate[T + t];
  for (int q = 1; q < ks; ++q) g += gate[T + q * T + t];
  gate[t] = sigmoid_f32(g);
}

// --------------------------------------------------------------------------
// scored routing with selection bias and optional group limit
// (ref/deepseek_v4.py:522-561; group limit per DeepSeek-V3 noaux_tc)
// --------------------------------------------------------------------------
enum Scoring { SCORE_SOFTMAX = 0, SCORE_SIGMOID = 1, SCORE_SQRTSOFTPLUS = 2 };

// Scores of one token's logits row on the calling wave (lane holds experts
// lane + 64 i): softmax in fp64 (ref/deepseek_v4.py:524-525), sigmoid in
// fp64 then fp32 (:526-528), sqrt(softplus) (:529-530, :534-537).
template <int EPL>
__device__ __forceinline__ void gate_scores_row(float* row, int ks,
                                                long kstride, bool store,
                                                int E, int scoring,
                                                float (&sc)[EPL]) {
  const int lane = threadIdx.x & 63;
  float lv[EPL];
  logit_sums<EPL>(row, ks, kstride, E, store, 0.f, lv);
  if (scoring == SCORE_SOFTMAX) {
    double m = -INFINITY;
    double xv[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      int e = lane + 64 * i;
      xv[i] = e < E ? (double)lv[i] : -INFINITY;
      m = xv[i] > m ? xv[i] : m;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      double q = __shfl_xor(m, o, kWave);
      m = q > m ? q : m;
    }
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      xv[i] = (lane + 64 * i) < E ? exp(xv[i] - m) : 0.0;
      s += xv[i];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
#pragma unroll
    for (int i = 0; i < EPL; ++i) sc[i] = (float)(xv[i] / s);
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      int e = lane + 64 * i;
      double xv = e < E ? (double)lv[i] : 0.0;
      if (scoring == SCORE_SIGMOID) {
        sc[i] = (float)(1.0 / (1.0 + exp(-xv)));
      } else {
        double sp = log1p(exp(-fabs(xv))) + (xv > 0.0 ? xv : 0.0);
        sc[i] = sqrtf((float)sp);
      }
    }
  }
}

// One token's scored routing on the calling wave: the row's scores
// (gate_scores_row) plus bias select; with n_group > 1 each group of
// E / n_group experts is scored by the sum of its two largest biased scores
// and the topk_group best groups are kept (ties: the lower group); the
// top-k of the kept experts' biased scores (ties: the lower id); the
// weights are their unbiased scores, renormalized over the picks unless
// softmax, times route_scale. sb, scl: this wave's LDS scratch of EPL * 64
// floats each. Lane j < topk writes slot j of w_row / id_row (both or
// neither non-null) and of id_lds (when non-null).
template <int EPL>
__device__ __forceinline__ void route_grouped_token(
    float* row, int ks, long kstride, bool store, int E, int topk, int n_group,
    int topk_group, int scoring, float route_scale,
    const float* __restrict__ bias, float* sb, float* scl,
    float* __restrict__ w_row, int* __restrict__ id_row, int* id_lds,
    float* w_lds = nullptr) {
  const int lane = threadIdx.x & 63;
  // the bias loads go out with the logits' (issued after the scores, they
  // added their latency: 1.6 us of the C4 in-launch routing)
  float bv[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    bv[i] = bias && e < E ? bias[e] : 0.f;
  }
  float sc[EPL];
  gate_scores_row<EPL>(row, ks, kstride, store, E, scoring, sc);
  float b[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    b[i] = e < E ? sc[i] + bv[i] : -INFINITY;
  }
  const bool keep_all = n_group <= 1;
  uint64_t gkeep = ~0ull;  // bit g set: group g kept (n_group <= 64)
  if (!keep_all) {
    const int gs = E / n_group;
    // group score = the sum of the group's two largest biased scores (NaN
    // never one of them, -inf when fewer than two others)
    uint64_t gkey = 0;
    if (gs <= 64 && (gs & (gs - 1)) == 0 && E % 64 == 0) {
      // a group is gs adjacent lanes of one register: (largest, second)
      // pairs merged across the group's lanes, NaN as -inf; the registers'
      // merges go step by step together, so that a step costs one shuffle
      // latency rather than one per register (C4: 3.0 -> 2.1 us)
      float m1[EPL], m2[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        m1[i] = b[i] == b[i] ? b[i] : -INFINITY;
        m2[i] = -INFINITY;
      }
      for (int o = 1; o < gs; o <<= 1) {
        float p1[EPL], p2[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          p1[i] = __shfl_xor(m1[i], o, kWave);
          p2[i] = __shfl_xor(m2[i], o, kWave);
        }
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          m2[i] = fmaxf(fminf(m1[i], p1[i]), fmaxf(m2[i], p2[i]));
          m1[i] = fmaxf(m1[i], p1[i]);
        }
      }
      // lane g of the wave takes group g = (64 i + lane') / gs from the
      // group's first lane lane'
      const int ng_i = 64 / gs;  // groups per register
      for (int q = 0; q < ng_i; ++q) {
        float v[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) v[i] = __shfl(m1[i] + m2[i], q * gs, kWave);
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const int g = i * ng_i + q;
          if (lane == g && g < n_group)
            gkey = ((uint64_t)f32_order_key(v[i]) << 32) |
                   (uint64_t)(0xFFFFFFFFu - (uint32_t)g);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (lane + 64 * i < E) sb[lane + 64 * i] = b[i];
      __builtin_amdgcn_wave_barrier();  // the wave's LDS accesses stay in order
      // lane g < n_group: its group's elements in turn
      if (lane < n_group) {
        float m1 = -INFINITY, m2 = -INFINITY;
        for (int q = 0; q < gs; ++q) {
          const float val = sb[lane * gs + q];
          if (val > m1) {
            m2 = m1;
            m1 = val;
          } else if (val > m2) {
            m2 = val;
          }
        }
        const float gsum = m1 + m2;
        gkey = ((uint64_t)f32_order_key(gsum) << 32) |
               (uint64_t)(0xFFFFFFFFu - (uint32_t)lane);
      }
    }
    gkeep = 0;
    for (int r = 0; r < topk_group; ++r) {
      const uint64_t best = wave_max_u64(gkey);
      const int g = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
      gkeep |= 1ull << g;
      if (lane == g) gkey = 0;
    }
  }
  uint64_t key[EPL];
  const int gs = keep_all ? E : E / n_group;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    const bool ok = e < E && (keep_all || ((gkeep >> (e / gs)) & 1ull));
    key[i] = ok ? topk_key(b[i], e) : 0ull;
    if (e < E) scl[e] = sc[i];  // the picks' unbiased scores, by id
  }
  __builtin_amdgcn_wave_barrier();
  const uint64_t pick = wave_topk_keys<EPL>(key, topk);
  const int myid = topk_key_id(pick);
  const float mine = lane < topk ? scl[min(max(myid, 0), E - 1)] : 0.f;
  float wsum = 0.f;
  for (int j = 0; j < topk; ++j)
    wsum += __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(mine), j));
  if (lane < topk) {
    const float wv = scoring == SCORE_SOFTMAX ? mine : mine / wsum;
    if (w_row) {
      w_row[lane] = wv * route_scale;
      id_row[lane] = myid;
    }
    if (id_lds) id_lds[lane] = myid;
    if (w_lds) w_lds[lane] = wv * route_scale;
  }
}

}  // namespace sllm
