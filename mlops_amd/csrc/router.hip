// Router kernels: top-k selection with route weights, routing statistics and
// the analytic logit gradient. One 64-lane wavefront owns one token; lane l
// holds experts l, l+64, ... so a token's logits are read once, coalesced.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {

constexpr int kMaxPerLane = 8;  // experts <= 512
constexpr int kMaxTopK = 32;
constexpr int kStatsChunk = 64;  // tokens per statistics chunk
constexpr int kTokensPerBlock = 4;

// Per-lane expert slots: unrolled so the arrays stay in registers.
#define SLOTS(i) _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) if (i < per_lane)

// Wave argmax with the stable-sort tie rule: larger value first, equal
// values -> smaller expert id. Returns the winning expert id (or -1).
__device__ __forceinline__ int wave_argmax(float v, int idx) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int oi = __shfl_xor(idx, o, 64);
    bool take = (oi >= 0) && (idx < 0 || ov > v || (ov == v && oi < idx));
    v = take ? ov : v;
    idx = take ? oi : idx;
  }
  return idx;
}

// Maximum over the wave, in every lane: within each row of 16 lanes by four
// DPP steps (quad swaps, then the half-row and row mirrors), then over the
// four rows' results read as scalars. No LDS round trips.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// One selection round: the best remaining eligible candidate of the wave
// (stable descending order: the largest value, ties to the lower expert id).
// `taken` is the lane's bitmask of used slots. Each lane keeps its best slot
// (the lower slot on ties); the wave maximum of those values comes from DPP
// steps, and the lanes holding it are found with one ballot per slot, slot 0
// first (ids lane + 64 * slot), lowest lane first. The winner is wave-uniform.
__device__ __forceinline__ int select_next(const float* val, const bool* eligible, int per_lane,
                                           uint32_t& taken) {
  const int lane = lane_id();
  float best = -INFINITY;
  int slot = -1;
  SLOTS(i) {
    if (!eligible[i] || ((taken >> i) & 1u)) continue;
    if (slot < 0 || val[i] > best) {  // ascending slot: strict > keeps the lower id
      best = val[i];
      slot = i;
    }
  }
  const float top = wave_max_dpp(slot >= 0 ? best : -INFINITY);
  int winner = -1;
  for (int s = 0; s < per_lane && winner < 0; ++s) {
    const uint64_t hit = __ballot(slot == s && best == top);
    if (hit != 0) winner = 64 * s + __builtin_ctzll(hit);
  }
  // No lane matched (only NaN values left): the lowest remaining id.
  for (int s = 0; s < per_lane && winner < 0; ++s) {
    const uint64_t any = __ballot(slot == s);
    if (any != 0) winner = 64 * s + __builtin_ctzll(any);
  }
  if (winner >= 0 && (winner & 63) == lane) taken |= 1u << (winner >> 6);
  return winner;
}

template <int PL>
__global__ void __launch_bounds__(256) router_topk_kernel(
    const float* __restrict__ logits, int tokens, int experts, int top_k, int mode,
    const float* __restrict__ bias, int n_group, int topk_group, float routed_scaling,
    const int32_t* __restrict__ forced, float* __restrict__ weights, int32_t* __restrict__ ids) {
  __shared__ float lds_sel[kTokensPerBlock][512];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int token = blockIdx.x * kTokensPerBlock + wave;
  if (token >= tokens) return;
  constexpr int per_lane = PL;  // slots per lane (experts <= 64 * PL)
  const float* row = logits + (size_t)token * experts;

  float l[kMaxPerLane], val[kMaxPerLane];
  bool ok[kMaxPerLane];
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) {
    int e = lane + 64 * i;
    l[i] = (i < per_lane && e < experts) ? row[e] : -INFINITY;
    ok[i] = (i < per_lane && e < experts);
  }

  // Full softmax (mode 1) or sigmoid scores (mode 2) where needed.
  float p[kMaxPerLane];
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) p[i] = 0.0f;
  if (mode == MI355X_ROUTE_SOFTMAX_THEN_TOPK) {
    float m = -INFINITY;
    SLOTS(i) m = fmaxf(m, l[i]);
    m = wave_max(m);
    float s = 0.0f;
    SLOTS(i) {
      p[i] = ok[i] ? __expf(l[i] - m) : 0.0f;
      s += p[i];
    }
    s = wave_sum(s);
    SLOTS(i) p[i] = p[i] / s;
  } else if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
    SLOTS(i) p[i] = ok[i] ? sigmoid_f(l[i]) : 0.0f;
  }

  if (forced == nullptr) {
    if (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) {
      SLOTS(i) val[i] = l[i];
    } else if (mode == MI355X_ROUTE_SOFTMAX_THEN_TOPK) {
      SLOTS(i) val[i] = p[i];
    } else {
      SLOTS(i) {
        int e = lane + 64 * i;
        val[i] = p[i] + (bias != nullptr && ok[i] ? bias[e] : 0.0f);
      }
      if (topk_group < n_group) {
        // Group-limited selection: a group's score is the sum of its two
        // largest selection values; keep the topk_group best groups.
        float* sv = lds_sel[wave];
        SLOTS(i) {
          int e = lane + 64 * i;
          if (e < experts) sv[e] = val[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int gsize = experts / n_group;
        float gscore = -INFINITY;
        if (lane < n_group) {
          float b1 = -INFINITY, b2 = -INFINITY;
          for (int t = 0; t < gsize; ++t) {
            float v = sv[lane * gsize + t];
            if (v > b1) { b2 = b1; b1 = v; } else if (v > b2) { b2 = v; }
          }
          gscore = gsize >= 2 ? b1 + b2 : b1;
        }
        uint64_t keep = 0;
        bool gtaken = false;
        for (int j = 0; j < topk_group; ++j) {
          int cand = (lane < n_group && !gtaken) ? lane : -1;
          int w = wave_argmax(gscore, cand);
          if (w >= 0) keep |= 1ull << w;
          if (w == lane) gtaken = true;
        }
        SLOTS(i) {
          int e = lane + 64 * i;
          if (e < experts && !((keep >> (e / gsize)) & 1ull)) val[i] = -INFINITY;
        }
      }
    }
  }

  // k rounds: pick (or read the forced) expert j, and hand its logit /
  // probability to lane j, which owns route weight j.
  uint32_t taken = 0;
  float mine = 0.0f;
  int my_id = 0;
  for (int j = 0; j < top_k; ++j) {
    int e = forced != nullptr ? forced[(size_t)token * top_k + j]
                              : select_next(val, ok, per_lane, taken);
    const int owner = __builtin_amdgcn_readfirstlane(e & 63), slot = e >> 6;
    float lv = 0.0f, pv = 0.0f;
    SLOTS(i) {
      if (i == slot) {
        lv = l[i];
        pv = p[i];
      }
    }
    lv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), owner));
    pv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), owner));
    if (lane == j) {
      mine = (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) ? lv : pv;
      my_id = e;
    }
  }
  float w = 0.0f;
  const bool active = lane < top_k;
  if (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) {
    float m = wave_max(active ? mine : -INFINITY);
    float ex = active ? __expf(mine - m) : 0.0f;
    float s = wave_sum(ex);
    w = ex / s;
  } else if (mode == MI355X_ROUTE_SOFTMAX_THEN_TOPK) {
    w = mine;
  } else {
    float s = wave_sum(active ? mine : 0.0f);
    w = mine / s * routed_scaling;
  }
  if (active) {
    weights[(size_t)token * top_k + lane] = w;
    ids[(size_t)token * top_k + lane] = my_id;
  }
}

// Per-chunk partial column sums of the routing probabilities and per-chunk
// expert counts. Wave w sums tokens start+w, start+w+4, ...; the four wave
// partials are then added in wave order, so the result is deterministic.
template <int PL>
__global__ void __launch_bounds__(256) router_stats_partial_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ ids, int tokens, int experts,
    int top_k, int mode, const int32_t* __restrict__ seg_offsets,
    const int32_t* __restrict__ chunk_table, float* __restrict__ part_p,
    int32_t* __restrict__ part_c) {
  __shared__ float wave_p[4][512];
  __shared__ int counts[512];
  const int c = blockIdx.x;
  int start, end;
  if (chunk_table == nullptr) {
    start = c * kStatsChunk;
    end = min(tokens, start + kStatsChunk);
  } else {
    start = chunk_table[2 * c];
    int seg = chunk_table[2 * c + 1];
    end = min(seg_offsets[seg + 1], start + kStatsChunk);
  }
  for (int e = threadIdx.x; e < experts; e += blockDim.x) counts[e] = 0;
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = lane_id();
  constexpr int per_lane = PL;  // slots per lane (experts <= 64 * PL)
  float acc[kMaxPerLane];
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) acc[i] = 0.0f;
  // The wave's tokens t = start + wave + 4u, four at a time: the four rows'
  // logits and route ids are loaded before any of them is used, then the
  // tokens are summed in order (the same order as one at a time).
  constexpr int kBatch = 4;
  for (int t0 = start + wave; t0 < end; t0 += 4 * kBatch) {
    float l[kBatch][kMaxPerLane];
    int id[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 4 * u;
      const float* row = logits + (size_t)t * experts;
      SLOTS(i) {
        int e = lane + 64 * i;
        l[u][i] = (t < end && e < experts) ? row[e] : -INFINITY;
      }
      id[u] = (t < end && lane < top_k) ? ids[(size_t)t * top_k + lane] : -1;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (t0 + 4 * u >= end) break;  // wave-uniform
      if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
        float s = 0.0f;
        SLOTS(i) {
          int e = lane + 64 * i;
          l[u][i] = e < experts ? sigmoid_f(l[u][i]) : 0.0f;
          s += l[u][i];
        }
        s = wave_sum(s);
        SLOTS(i) acc[i] += l[u][i] / s;
      } else {
        float m = -INFINITY;
        SLOTS(i) m = fmaxf(m, l[u][i]);
        m = wave_max(m);
        float s = 0.0f;
        SLOTS(i) {
          l[u][i] = (lane + 64 * i) < experts ? __expf(l[u][i] - m) : 0.0f;
          s += l[u][i];
        }
        s = wave_sum(s);
        SLOTS(i) acc[i] += l[u][i] / s;
      }
      if (id[u] >= 0) atomicAdd(&counts[id[u]], 1);
    }
  }
  SLOTS(i) {
    int e = lane + 64 * i;
    if (e < experts) wave_p[wave][e] = acc[i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    float s = ((wave_p[0][e] + wave_p[1][e]) + wave_p[2][e]) + wave_p[3][e];
    part_p[(size_t)c * experts + e] = s;
    part_c[(size_t)c * experts + e] = counts[e];
  }
}

// Reduce the chunk partials per segment (in chunk order), then the aux loss.
__global__ void __launch_bounds__(256) router_stats_final_kernel(
    const float* __restrict__ part_p, const int32_t* __restrict__ part_c, int nchunks,
    int tokens, int experts, int top_k, int mode, int segments,
    const int32_t* __restrict__ seg_offsets, const int32_t* __restrict__ chunk_table,
    float* __restrict__ aux, float* __restrict__ prob_sum, int32_t* __restrict__ seg_counts) {
  __shared__ float red[256];
  float aux_part = 0.0f;
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    float total_p = 0.0f;
    int total_c = 0;
    int c = 0;
    for (int s = 0; s < segments; ++s) {
      float sp = 0.0f;
      int sc = 0;
      while (c < nchunks) {
        int seg = chunk_table == nullptr ? 0 : chunk_table[2 * c + 1];
        if (seg != s) break;
        sp += part_p[(size_t)c * experts + e];
        sc += part_c[(size_t)c * experts + e];
        ++c;
      }
      seg_counts[(size_t)s * experts + e] = sc;
      total_p += sp;
      total_c += sc;
      if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
        int len = seg_offsets == nullptr ? tokens : seg_offsets[s + 1] - seg_offsets[s];
        float freq = (float)sc * (float)experts / (float)(top_k * len);
        aux_part += freq * (sp / (float)len);
      }
    }
    prob_sum[e] = total_p;
    if (mode != MI355X_ROUTE_SIGMOID_NOAUX_TC) {
      // softmax modes: one aux over all rows, whatever the segments
      float freq = (float)total_c / (float)(tokens * top_k);
      aux_part += freq * (total_p / (float)tokens);
    }
  }
  red[threadIdx.x] = aux_part;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0)
    aux[0] = mode == MI355X_ROUTE_SIGMOID_NOAUX_TC ? red[0] : (float)experts * red[0];
}

// Parallel form of the final reduction: each (segment, expert) sum is spread
// over G lanes of one wave (chunks part, part + G, ...), reduced by a fixed
// butterfly, so results are deterministic. Sizes beyond the LDS tables use the
// serial kernel above.
constexpr int kReduceThreads = 1024;
constexpr int kReduceMaxSegments = 1024;
constexpr int kReduceMaxPairs = 8192;

__global__ void __launch_bounds__(kReduceThreads) router_stats_reduce_kernel(
    const float* __restrict__ part_p, const int32_t* __restrict__ part_c, int nchunks,
    int tokens, int experts, int top_k, int mode, int segments,
    const int32_t* __restrict__ seg_offsets, const int32_t* __restrict__ chunk_table,
    float* __restrict__ aux, float* __restrict__ prob_sum, int32_t* __restrict__ seg_counts) {
  __shared__ int seg_start[kReduceMaxSegments + 1];
  __shared__ float sp_lds[kReduceMaxPairs];
  __shared__ int sc_lds[kReduceMaxPairs];
  __shared__ float red[kReduceThreads / 64];
  const int tid = threadIdx.x;
  // First chunk of every segment (chunks are ordered by segment).
  if (chunk_table == nullptr) {
    if (tid == 0) {
      seg_start[0] = 0;
      seg_start[1] = nchunks;
    }
  } else {
    for (int c = tid; c < nchunks; c += kReduceThreads) {
      const int s = chunk_table[2 * c + 1];
      const int prev = c == 0 ? -1 : chunk_table[2 * c - 1];
      for (int q = prev + 1; q <= s; ++q) seg_start[q] = c;
      if (c == nchunks - 1)
        for (int q = s + 1; q <= segments; ++q) seg_start[q] = nchunks;
    }
  }
  __syncthreads();
  const int pairs = segments * experts;
  int G = 64;
  while (G > 1 && pairs * G > kReduceThreads) G >>= 1;
  for (int base = 0; base < pairs * G; base += kReduceThreads) {
    const int idx = base + tid;
    const int pair = idx / G, part = idx % G;
    float sp = 0.0f;
    int sc = 0;
    if (pair < pairs) {
      const int seg = pair / experts, e = pair % experts;
      // Sixteen chunks' partials are loaded before they are summed (in order).
      constexpr int kBatch = 16;
      const int c_end = seg_start[seg + 1];
      for (int c0 = seg_start[seg] + part; c0 < c_end; c0 += kBatch * G) {
        float pv[kBatch];
        int cv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int c = c0 + j * G;
          pv[j] = c < c_end ? part_p[(size_t)c * experts + e] : 0.0f;
          cv[j] = c < c_end ? part_c[(size_t)c * experts + e] : 0;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          sp += pv[j];
          sc += cv[j];
        }
      }
    }
    for (int o = G >> 1; o >= 1; o >>= 1) {
      sp += __shfl_xor(sp, o, 64);
      sc += __shfl_xor(sc, o, 64);
    }
    if (pair < pairs && part == 0) {
      sp_lds[pair] = sp;
      sc_lds[pair] = sc;
      seg_counts[pair] = sc;
    }
  }
  __syncthreads();
  float aux_part = 0.0f;
  for (int e = tid; e < experts; e += kReduceThreads) {
    float total_p = 0.0f;
    int total_c = 0;
    for (int s = 0; s < segments; ++s) {
      const float sp = sp_lds[s * experts + e];
      total_p += sp;
      total_c += sc_lds[s * experts + e];
      if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
        const int len = seg_offsets == nullptr ? tokens : seg_offsets[s + 1] - seg_offsets[s];
        const float freq = (float)sc_lds[s * experts + e] * (float)experts / (float)(top_k * len);
        aux_part += freq * (sp / (float)len);
      }
    }
    prob_sum[e] = total_p;
    if (mode != MI355X_ROUTE_SIGMOID_NOAUX_TC) {
      // softmax modes: one aux over all rows, whatever the segments
      const float freq = (float)total_c / (float)(tokens * top_k);
      aux_part += freq * (total_p / (float)tokens);
    }
  }
  aux_part = wave_sum(aux_part);
  if (lane_id() == 0) red[tid >> 6] = aux_part;
  __syncthreads();
  if (tid == 0) {
    float total = 0.0f;
    for (int w = 0; w < kReduceThreads / 64; ++w) total += red[w];
    aux[0] = mode == MI355X_ROUTE_SIGMOID_NOAUX_TC ? total : (float)experts * total;
  }
}

template <int PL>
__global__ void __launch_bounds__(256) router_bwd_kernel(
    const float* __restrict__ logits, const float* __restrict__ weights,
    const int32_t* __restrict__ ids, const float* __restrict__ dscore,
    const int32_t* __restrict__ slots, int tokens, int experts, int top_k, int mode,
    const float* __restrict__ grad_aux, const float* __restrict__ grad_ps,
    const int32_t* __restrict__ offsets, int segments, const int32_t* __restrict__ seg_offsets,
    const int32_t* __restrict__ seg_counts, float* __restrict__ grad_logits, uint16_t* __restrict__ pieces) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int token = blockIdx.x * kTokensPerBlock + wave;
  if (token >= tokens) return;
  constexpr int per_lane = PL;  // slots per lane (experts <= 64 * PL)
  const float* row = logits + (size_t)token * experts;
  float l[kMaxPerLane], g[kMaxPerLane];
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) {
    int e = lane + 64 * i;
    l[i] = (i < per_lane && e < experts) ? row[e] : -INFINITY;
    g[i] = 0.0f;
  }
  // Route-weight cotangent of this token's k choices (lane j owns choice j).
  const bool active = lane < top_k;
  float gw = 0.0f, wj = 0.0f;
  int idj = 0;
  if (active) {
    size_t flat = (size_t)token * top_k + lane;
    gw = dscore[slots[flat]];
    wj = weights[flat];
    idj = ids[flat];
  }
  // Probabilities of the token (softmax or normalized sigmoid).
  float p[kMaxPerLane], s[kMaxPerLane];
  if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
    float rs = 0.0f;
    SLOTS(i) {
      s[i] = (lane + 64 * i) < experts ? sigmoid_f(l[i]) : 0.0f;
      rs += s[i];
    }
    rs = wave_sum(rs);
    SLOTS(i) p[i] = s[i] / rs;
    // route_backward, sigmoid branch (moe_router.py:406-421).
    float sj = active ? sigmoid_f(row[idj]) : 0.0f;
    float score_sum = wave_sum(sj);
    float scaling = wave_sum(active ? wj : 0.0f);
    float dot = wave_sum(active ? gw * wj : 0.0f);
    float selg = active ? ((scaling * gw - dot) / score_sum) * sj * (1.0f - sj) : 0.0f;
    for (int j = 0; j < top_k; ++j) {
      float v = __shfl(selg, j, 64);
      int e = __shfl(idj, j, 64);
      SLOTS(i)
        if (e == lane + 64 * i) g[i] += v;
    }
    // Per-sequence aux gradient (moe_router.py:476-502).
    if (grad_aux != nullptr) {
      int seg = 0;
      if (seg_offsets != nullptr) {
        int lo = 0, hi = segments - 1;
        while (lo < hi) {
          int mid = (lo + hi + 1) >> 1;
          if (seg_offsets[mid] <= token) lo = mid; else hi = mid - 1;
        }
        seg = lo;
      }
      int len = seg_offsets == nullptr ? tokens : seg_offsets[seg + 1] - seg_offsets[seg];
      float f[kMaxPerLane];
      float qf = 0.0f;
      SLOTS(i) {
        int e = lane + 64 * i;
        f[i] = e < experts ? (float)seg_counts[(size_t)seg * experts + e] * (float)experts /
                                 (float)(top_k * len)
                           : 0.0f;
        qf += p[i] * f[i];
      }
      qf = wave_sum(qf);
      float coef = grad_aux[0] / ((float)len * rs);
      SLOTS(i) g[i] += coef * (f[i] - qf) * s[i] * (1.0f - s[i]);
    }
    if (grad_ps != nullptr) {
      float pg = 0.0f;
      SLOTS(i) {
        int e = lane + 64 * i;
        pg += e < experts ? p[i] * grad_ps[e] : 0.0f;
      }
      pg = wave_sum(pg);
      SLOTS(i) {
        int e = lane + 64 * i;
        if (e < experts) g[i] += (1.0f - s[i]) * p[i] * (grad_ps[e] - pg);
      }
    }
  } else {
    float m = -INFINITY;
    SLOTS(i) m = fmaxf(m, l[i]);
    m = wave_max(m);
    float z = 0.0f;
    SLOTS(i) {
      p[i] = (lane + 64 * i) < experts ? __expf(l[i] - m) : 0.0f;
      z += p[i];
    }
    z = wave_sum(z);
    SLOTS(i) p[i] = p[i] / z;
    if (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) {
      // p_sel (g - <g, p_sel>) scattered to the chosen experts.
      float dot = wave_sum(active ? gw * wj : 0.0f);
      float v = active ? wj * (gw - dot) : 0.0f;
      for (int j = 0; j < top_k; ++j) {
        float vj = __shfl(v, j, 64);
        int e = __shfl(idj, j, 64);
        SLOTS(i)
          if (e == lane + 64 * i) g[i] += vj;
      }
    } else {
      // -p * <g, p_sel> + scatter(g * p_sel).
      float psel = 0.0f;
      for (int j = 0; j < top_k; ++j) {
        int e = __shfl(idj, j, 64);
        float pe = 0.0f;
        SLOTS(i)
          if (e == lane + 64 * i) pe = p[i];
        pe = __shfl(pe, e & 63, 64);
        if (lane == j) psel = pe;
      }
      float dot = wave_sum(active ? gw * psel : 0.0f);
      SLOTS(i) g[i] = -p[i] * dot;
      float v = active ? gw * psel : 0.0f;
      for (int j = 0; j < top_k; ++j) {
        float vj = __shfl(v, j, 64);
        int e = __shfl(idj, j, 64);
        SLOTS(i)
          if (e == lane + 64 * i) g[i] += vj;
      }
    }
    // Batch aux gradient (moe_router.py:455-473): c * p (f - <p, f>).
    if (grad_aux != nullptr) {
      float f[kMaxPerLane];
      float pf = 0.0f;
      SLOTS(i) {
        int e = lane + 64 * i;
        f[i] = e < experts ? (float)(offsets[e + 1] - offsets[e]) / (float)(tokens * top_k) : 0.0f;
        pf += p[i] * f[i];
      }
      pf = wave_sum(pf);
      float coef = grad_aux[0] * (float)experts / (float)tokens;
      SLOTS(i) g[i] += coef * p[i] * (f[i] - pf);
    }
    if (grad_ps != nullptr) {
      float pg = 0.0f;
      SLOTS(i) {
        int e = lane + 64 * i;
        pg += e < experts ? p[i] * grad_ps[e] : 0.0f;
      }
      pg = wave_sum(pg);
      SLOTS(i) {
        int e = lane + 64 * i;
        if (e < experts) g[i] += p[i] * (grad_ps[e] - pg);
      }
    }
  }
  if (grad_logits != nullptr) {
    float* out = grad_logits + (size_t)token * experts;
    SLOTS(i) {
      int e = lane + 64 * i;
      if (e < experts) out[e] = g[i];
    }
  }
  if (pieces != nullptr) {
    // The two bf16 pieces of the router weight gradient's operand, side by
    // side in a row of 2E: hi = bf16(g), mid = bf16(g - hi) (both rounded to
    // nearest even, as torch's casts).
    uint16_t* row_out = pieces + (size_t)token * 2 * experts;
    SLOTS(i) {
      int e = lane + 64 * i;
      if (e < experts) {
        const uint16_t hi = f32_to_bf16(g[i]);
        row_out[e] = hi;
        row_out[experts + e] = f32_to_bf16(g[i] - bf16_to_f32(hi));
      }
    }
  }
}

// Expert slots per lane the kernels are compiled for: the smallest of 1, 2,
// 4 and 8 that covers ceil(experts / 64) (slots past `experts` are masked).
int slots_per_lane(int experts) {
  const int need = (experts + 63) / 64;
  return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
}

}  // namespace

extern "C" int mi355x_router_topk(const float* logits, int tokens, int experts, int top_k,
                                  int mode, const float* bias, int n_group, int topk_group,
                                  float routed_scaling, const int32_t* forced_ids,
                                  float* weights, int32_t* ids, void* stream) {
  MI355X_REQUIRE(tokens >= 0 && experts > 0 && experts <= 64 * kMaxPerLane,
                 "router: experts must be in [1, %d], got %d", 64 * kMaxPerLane, experts);
  MI355X_REQUIRE(top_k > 0 && top_k <= experts && top_k <= kMaxTopK,
                 "router: top_k must be in [1, min(E, %d)], got %d", kMaxTopK, top_k);
  MI355X_REQUIRE(mode >= 0 && mode <= 2, "router: unknown mode %d", mode);
  if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
    MI355X_REQUIRE(n_group > 0 && experts % n_group == 0 && n_group <= 64,
                   "router: n_group must divide experts and be <= 64");
    MI355X_REQUIRE(topk_group > 0, "router: topk_group must be positive");
  }
  if (tokens == 0) return MI355X_OK;
  dim3 grid((tokens + kTokensPerBlock - 1) / kTokensPerBlock);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, (hipStream_t)stream, logits, tokens, experts,
                       top_k, mode, bias, n_group, topk_group, routed_scaling, forced_ids,
                       weights, ids);
  };
  switch (slots_per_lane(experts)) {
    case 1: launch(router_topk_kernel<1>); break;
    case 2: launch(router_topk_kernel<2>); break;
    case 4: launch(router_topk_kernel<4>); break;
    default: launch(router_topk_kernel<8>); break;
  }
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" size_t mi355x_router_stats_workspace_size(int nchunks, int experts) {
  size_t n = (size_t)nchunks * experts;
  return n * sizeof(float) + n * sizeof(int32_t) + 256;
}

extern "C" int mi355x_router_stats(const float* logits, const int32_t* ids, int tokens,
                                   int experts, int top_k, int mode, int segments,
                                   const int32_t* seg_offsets, const int32_t* chunk_table,
                                   int nchunks, float* aux, float* prob_sum, int32_t* seg_counts,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= 64 * kMaxPerLane, "router_stats: bad experts %d",
                 experts);
  MI355X_REQUIRE(tokens > 0 && top_k > 0 && top_k <= 64, "router_stats: bad tokens/top_k");
  MI355X_REQUIRE(segments >= 1, "router_stats: segments must be >= 1");
  if (chunk_table == nullptr) {
    MI355X_REQUIRE(segments == 1, "router_stats: several segments need a chunk table");
    MI355X_REQUIRE(nchunks == (tokens + kStatsChunk - 1) / kStatsChunk,
                   "router_stats: nchunks must be ceil(tokens / %d)", kStatsChunk);
  } else {
    MI355X_REQUIRE(seg_offsets != nullptr, "router_stats: chunk table needs seg_offsets");
  }
  MI355X_REQUIRE(workspace_bytes >= mi355x_router_stats_workspace_size(nchunks, experts),
                 "router_stats: workspace too small");
  float* part_p = (float*)workspace;
  int32_t* part_c = (int32_t*)(part_p + (size_t)nchunks * experts);
  hipStream_t s = (hipStream_t)stream;
  auto partial = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(nchunks), dim3(256), 0, s, logits, ids, tokens, experts, top_k,
                       mode, seg_offsets, chunk_table, part_p, part_c);
  };
  switch (slots_per_lane(experts)) {
    case 1: partial(router_stats_partial_kernel<1>); break;
    case 2: partial(router_stats_partial_kernel<2>); break;
    case 4: partial(router_stats_partial_kernel<4>); break;
    default: partial(router_stats_partial_kernel<8>); break;
  }
  MI355X_LAUNCH_CHECK();
  if (segments <= kReduceMaxSegments && (size_t)segments * experts <= kReduceMaxPairs) {
    hipLaunchKernelGGL(router_stats_reduce_kernel, dim3(1), dim3(kReduceThreads), 0, s, part_p,
                       part_c, nchunks, tokens, experts, top_k, mode, segments, seg_offsets,
                       chunk_table, aux, prob_sum, seg_counts);
  } else {
    hipLaunchKernelGGL(router_stats_final_kernel, dim3(1), dim3(256), 0, s, part_p, part_c,
                       nchunks, tokens, experts, top_k, mode, segments, seg_offsets, chunk_table,
                       aux, prob_sum, seg_counts);
  }
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

namespace {
int router_bwd_launch(const float* logits, const float* weights, const int32_t* ids,
                      const float* dscore, const int32_t* slots, int tokens, int experts,
                      int top_k, int mode, const float* grad_aux, const float* grad_prob_sum,
                      const int32_t* offsets, int segments, const int32_t* seg_offsets,
                      const int32_t* seg_counts, float* grad_logits, uint16_t* pieces,
                      void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= 64 * kMaxPerLane, "router_bwd: bad experts %d",
                 experts);
  MI355X_REQUIRE(top_k > 0 && top_k <= experts && top_k <= kMaxTopK, "router_bwd: bad top_k");
  MI355X_REQUIRE(mode >= 0 && mode <= 2, "router_bwd: unknown mode %d", mode);
  if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC && grad_aux != nullptr)
    MI355X_REQUIRE(seg_counts != nullptr && (segments == 1 || seg_offsets != nullptr),
                   "router_bwd: sequence aux gradient needs segment counts and offsets");
  if (mode != MI355X_ROUTE_SIGMOID_NOAUX_TC && grad_aux != nullptr)
    MI355X_REQUIRE(offsets != nullptr, "router_bwd: aux gradient needs expert offsets");
  if (tokens == 0) return MI355X_OK;
  dim3 grid((tokens + kTokensPerBlock - 1) / kTokensPerBlock);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, (hipStream_t)stream, logits, weights, ids,
                       dscore, slots, tokens, experts, top_k, mode, grad_aux, grad_prob_sum,
                       offsets, segments, seg_offsets, seg_counts, grad_logits, pieces);
  };
  switch (slots_per_lane(experts)) {
    case 1: launch(router_bwd_kernel<1>); break;
    case 2: launch(router_bwd_kernel<2>); break;
    case 4: launch(router_bwd_kernel<4>); break;
    default: launch(router_bwd_kernel<8>); break;
  }
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
}  // namespace

extern "C" int mi355x_router_topk_bwd(const float* logits, const float* weights,
                                      const int32_t* ids, const float* dscore,
                                      const int32_t* slots, int tokens, int experts, int top_k,
                                      int mode, const float* grad_aux, const float* grad_prob_sum,
                                      const int32_t* offsets, int segments,
                                      const int32_t* seg_offsets, const int32_t* seg_counts,
                                      float* grad_logits, void* stream) {
  MI355X_REQUIRE(grad_logits != nullptr, "router_bwd: grad_logits is required");
  return router_bwd_launch(logits, weights, ids, dscore, slots, tokens, experts, top_k, mode,
                           grad_aux, grad_prob_sum, offsets, segments, seg_offsets, seg_counts,
                           grad_logits, nullptr, stream);
}

extern "C" int mi355x_router_topk_bwd_split(const float* logits, const float* weights,
                                            const int32_t* ids, const float* dscore,
                                            const int32_t* slots, int tokens, int experts,
                                            int top_k, int mode, const float* grad_aux,
                                            const float* grad_prob_sum, const int32_t* offsets,
                                            int segments, const int32_t* seg_offsets,
                                            const int32_t* seg_counts, float* grad_logits,
                                            void* pieces, void* stream) {
  MI355X_REQUIRE(pieces != nullptr, "router_bwd_split: the bf16 pieces output is required");
  return router_bwd_launch(logits, weights, ids, dscore, slots, tokens, experts, top_k, mode,
                           grad_aux, grad_prob_sum, offsets, segments, seg_offsets, seg_counts,
                           grad_logits, (uint16_t*)pieces, stream);
}
