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
// A token belongs to a group of W lanes: W = 64 (a wavefront) in general,
// W = 16 (four tokens per wavefront) when experts <= 128 and top_k <= 16.
// Lane l of a group holds experts l, l + W, ...; every reduction over a
// token's experts stays inside its group (DPP row steps for W = 16), so the
// narrow form spends a quarter of the instructions per token.
constexpr int kRowExperts = 128;
constexpr int kRowTopK = 16;

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

// Maximum of a uint32 over a group of W lanes, in every lane of the group
// (DPP row steps fused into v_max_u32; a source lane outside the row or not
// active reads as 0, the identity).
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_max_u32_step(uint32_t v) {
  return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, true));
}
template <int W>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  v = dpp_max_u32_step<0xB1>(v);
  v = dpp_max_u32_step<0x4E>(v);
  v = dpp_max_u32_step<0x141>(v);
  v = dpp_max_u32_step<0x140>(v);
#pragma unroll
  for (int o = 16; o < W; o <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}

// Selection key of a candidate: larger key = earlier in torch's stable
// descending sort. Numbers keep their order (-0 and +0 equal), NaN comes
// before every number (as torch.sort places it), and 0 marks a slot that is
// not (or no longer) a candidate; -inf maps to 0x007fffff, above it.
__device__ __forceinline__ uint32_t selection_key(float v) {
  if (v != v) return 0xffffffffu;
  const uint32_t b = __float_as_uint(v + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Top-k over a token's W-lane group. Each lane keeps the best of its own
// remaining slots (key, then the lower slot); a round takes the group's
// largest key by DPP steps and, among the lanes holding it, the lowest
// expert id by a group minimum. Only the winning lane's best changes, so
// the per-lane scan runs once up front and once per round for the winner's
// lane. The winner's logit and probability travel with its best.
template <int W, int PL>
struct LaneBest {
  uint32_t key[kMaxPerLane];
  uint32_t bk;
  int bs;
  float bl, bp;
  __device__ __forceinline__ void scan(const float* l, const float* p) {
    constexpr int per_lane = PL;
    bk = 0;
    bs = 0;
    bl = l[0];
    bp = p[0];
    SLOTS(i) {
      const bool better = key[i] > bk;  // strict: ties keep the lower slot
      bk = better ? key[i] : bk;
      bs = better ? i : bs;
      bl = better ? l[i] : bl;
      bp = better ? p[i] : bp;
    }
  }
};

template <int W, int PL>
__global__ void __launch_bounds__(256) router_topk_kernel(
    const float* __restrict__ logits, int tokens, int experts, int top_k, int mode,
    const float* __restrict__ bias, int n_group, int topk_group, float routed_scaling,
    const int32_t* __restrict__ forced, float* __restrict__ weights, int32_t* __restrict__ ids) {
  __shared__ float lds_sel[W == 64 ? 4 : 1][W == 64 ? 512 : 1];
  const int lane = threadIdx.x & (W - 1), gbase = lane_id() & ~(W - 1);
  const int token = blockIdx.x * (256 / W) + threadIdx.x / W;
  if (token >= tokens) return;
  constexpr int per_lane = PL;  // slots per lane (experts <= W * PL)
  const float* row = logits + (size_t)token * experts;

  float l[kMaxPerLane], val[kMaxPerLane];
  bool ok[kMaxPerLane];
  // Loads from clamped indices, unconditionally, so that none waits inside a
  // branch; slots past `experts` are masked afterwards.
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) {
    int e = lane + W * i;
    float x = -INFINITY;
    if (i < per_lane) x = row[min(e, experts - 1)];
    ok[i] = (i < per_lane && e < experts);
    l[i] = ok[i] ? x : -INFINITY;
  }

  // Full softmax (mode 1) or sigmoid scores (mode 2) where needed.
  float p[kMaxPerLane];
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) p[i] = 0.0f;
  if (mode == MI355X_ROUTE_SOFTMAX_THEN_TOPK) {
    float m = -INFINITY;
    SLOTS(i) m = fmaxf(m, l[i]);
    m = group_max<W>(m);
    float s = 0.0f;
    SLOTS(i) {
      p[i] = ok[i] ? __expf(l[i] - m) : 0.0f;
      s += p[i];
    }
    s = group_sum<W>(s);
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
        int e = lane + W * i;
        const float b = bias != nullptr ? bias[min(e, experts - 1)] : 0.0f;
        val[i] = p[i] + (ok[i] ? b : 0.0f);
      }
      if constexpr (W == 64) {
        if (topk_group < n_group) {
          // Group-limited selection: a group's score is the sum of its two
          // largest selection values; keep the topk_group best groups.
          float* sv = lds_sel[threadIdx.x >> 6];
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
  }

  // k rounds: pick (or read the forced) expert j, and hand its logit /
  // probability to lane j of the group, which owns route weight j.
  float mine = 0.0f;
  int my_id = 0;
  if (forced != nullptr) {
    for (int j = 0; j < top_k; ++j) {
      const int e = forced[(size_t)token * top_k + j];
      const int slot = e / W;
      float lv = 0.0f, pv = 0.0f;
      SLOTS(i) {
        if (i == slot) {
          lv = l[i];
          pv = p[i];
        }
      }
      const int owner = gbase + e % W;
      lv = __shfl(lv, owner, 64);
      pv = __shfl(pv, owner, 64);
      if (lane == j) {
        mine = (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) ? lv : pv;
        my_id = e;
      }
    }
  } else {
    LaneBest<W, PL> lb;
    SLOTS(i) lb.key[i] = ok[i] ? selection_key(val[i]) : 0u;
    lb.scan(l, p);
    for (int j = 0; j < top_k; ++j) {
      const uint32_t top = group_max_u32<W>(lb.bk);
      // The lowest id holding the top key, as the maximum of ~id.
      const int e = (int)~group_max_u32<W>(lb.bk == top && top != 0u ? ~(uint32_t)(W * lb.bs + lane)
                                                                     : 0u);
      const int owner = gbase + e % W;
      const float lv = __shfl(lb.bl, owner, 64), pv = __shfl(lb.bp, owner, 64);
      if (lane == j) {
        mine = (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) ? lv : pv;
        my_id = e;
      }
      if (e % W == lane) {
        SLOTS(i) if (i == lb.bs) lb.key[i] = 0u;
        lb.scan(l, p);
      }
    }
  }
  float w = 0.0f;
  const bool active = lane < top_k;
  if (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) {
    float m = group_max<W>(active ? mine : -INFINITY);
    float ex = active ? __expf(mine - m) : 0.0f;
    float s = group_sum<W>(ex);
    w = ex / s;
  } else if (mode == MI355X_ROUTE_SOFTMAX_THEN_TOPK) {
    w = mine;
  } else {
    float s = group_sum<W>(active ? mine : 0.0f);
    w = mine / s * routed_scaling;
  }
  if (active) {
    weights[(size_t)token * top_k + lane] = w;
    ids[(size_t)token * top_k + lane] = my_id;
  }
}

// Per-chunk partial column sums of the routing probabilities and per-chunk
// expert counts. Group q of the block sums tokens start+q, start+q+G, ...
// (G = 256 / W groups); the G group partials are then added in group order,
// so the result is deterministic.
template <int W, int PL>
__global__ void __launch_bounds__(256) router_stats_partial_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ ids, int tokens, int experts,
    int top_k, int mode, const int32_t* __restrict__ seg_offsets,
    const int32_t* __restrict__ chunk_table, float* __restrict__ part_p,
    int32_t* __restrict__ part_c) {
  constexpr int G = 256 / W;
  __shared__ float grp_p[G][W * PL];
  __shared__ int counts[W * PL];
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
  const int grp = threadIdx.x / W, lane = threadIdx.x & (W - 1);
  constexpr int per_lane = PL;  // slots per lane (experts <= W * PL)
  float acc[kMaxPerLane];
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) acc[i] = 0.0f;
  // The group's tokens t = start + grp + G u, four at a time: the four rows'
  // logits and route ids are loaded before any of them is used, then the
  // tokens are summed in order (the same order as one at a time).
  constexpr int kBatch = 4;
  for (int t0 = start + grp; t0 < end; t0 += G * kBatch) {
    float l[kBatch][kMaxPerLane];
    int id[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + G * u;
      const float* row = logits + (size_t)t * experts;
      SLOTS(i) {
        int e = lane + W * i;
        l[u][i] = (t < end && e < experts) ? row[e] : -INFINITY;
      }
      id[u] = (t < end && lane < top_k) ? ids[(size_t)t * top_k + lane] : -1;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (t0 + G * u >= end) break;  // uniform over the group
      if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
        float s = 0.0f;
        SLOTS(i) {
          int e = lane + W * i;
          l[u][i] = e < experts ? sigmoid_f(l[u][i]) : 0.0f;
          s += l[u][i];
        }
        s = group_sum<W>(s);
        SLOTS(i) acc[i] += l[u][i] / s;
      } else {
        float m = -INFINITY;
        SLOTS(i) m = fmaxf(m, l[u][i]);
        m = group_max<W>(m);
        float s = 0.0f;
        SLOTS(i) {
          l[u][i] = (lane + W * i) < experts ? __expf(l[u][i] - m) : 0.0f;
          s += l[u][i];
        }
        s = group_sum<W>(s);
        SLOTS(i) acc[i] += l[u][i] / s;
      }
      if (id[u] >= 0) atomicAdd(&counts[id[u]], 1);
    }
  }
  SLOTS(i) {
    int e = lane + W * i;
    if (e < experts) grp_p[grp][e] = acc[i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    float s = grp_p[0][e];
#pragma unroll
    for (int q = 1; q < G; ++q) s += grp_p[q][e];
    part_p[(size_t)c * experts + e] = s;
    part_c[(size_t)c * experts + e] = counts[e];
  }
}

// Reduce the chunk partials per segment (in chunk order), then the aux loss.
// Serial form, for segment counts beyond the LDS tables of the parallel one.
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

// Parallel form of the final reduction, in two kernels.
constexpr int kReduceMaxSegments = 1024;
constexpr int kPairLanes = 16;  // lanes per (segment, expert) sum

// First chunk of every segment (chunks are ordered by segment) into LDS.
__device__ void segment_starts(const int32_t* __restrict__ chunk_table, int nchunks,
                               int segments, int* seg_start) {
  if (chunk_table == nullptr) {
    if (threadIdx.x == 0) {
      seg_start[0] = 0;
      seg_start[1] = nchunks;
    }
  } else {
    for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
      const int s = chunk_table[2 * c + 1];
      const int prev = c == 0 ? -1 : chunk_table[2 * c - 1];
      for (int q = prev + 1; q <= s; ++q) seg_start[q] = c;
      if (c == nchunks - 1)
        for (int q = s + 1; q <= segments; ++q) seg_start[q] = nchunks;
    }
  }
  __syncthreads();
}

// 1. Each (segment, expert) pair's chunk partials summed by 16 lanes (chunks
//    part, part + 16, ... in order, then a fixed butterfly), so the result
//    is deterministic. The count goes to seg_counts; the probability sum is
//    written over the segment's first chunk partial, which only this pair
//    reads.
__global__ void __launch_bounds__(256) router_stats_pairs_kernel(
    float* __restrict__ part_p, const int32_t* __restrict__ part_c, int nchunks, int experts,
    int segments, const int32_t* __restrict__ chunk_table, int32_t* __restrict__ seg_counts) {
  __shared__ int seg_start[kReduceMaxSegments + 1];
  segment_starts(chunk_table, nchunks, segments, seg_start);
  const int pair = blockIdx.x * (256 / kPairLanes) + threadIdx.x / kPairLanes;
  const int part = threadIdx.x % kPairLanes;
  const int pairs = segments * experts;
  if (pair >= pairs) return;  // whole 16-lane groups
  const int seg = pair / experts, e = pair % experts;
  const int c0 = seg_start[seg], c_end = seg_start[seg + 1];
  float sp = 0.0f;
  int sc = 0;
  constexpr int kBatch = 16;  // loads issued before they are summed (in order)
  for (int cb = c0 + part; cb < c_end; cb += kBatch * kPairLanes) {
    float pv[kBatch];
    int cv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int c = cb + j * kPairLanes;
      pv[j] = c < c_end ? part_p[(size_t)c * experts + e] : 0.0f;
      cv[j] = c < c_end ? part_c[(size_t)c * experts + e] : 0;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      sp += pv[j];
      sc += cv[j];
    }
  }
  sp = group_sum<kPairLanes>(sp);
#pragma unroll
  for (int o = kPairLanes / 2; o >= 1; o >>= 1) sc += __shfl_xor(sc, o, 64);
  if (part == 0) {
    seg_counts[pair] = sc;
    if (c0 < c_end) part_p[(size_t)c0 * experts + e] = sp;
  }
}

// 2. Per expert: the segment sums into prob_sum and the aux loss terms, added
//    over experts in a fixed order.
constexpr int kAuxThreads = 512;
__global__ void __launch_bounds__(kAuxThreads) router_stats_aux_kernel(
    const float* __restrict__ part_p, int nchunks, int tokens, int experts, int top_k, int mode,
    int segments, const int32_t* __restrict__ seg_offsets,
    const int32_t* __restrict__ chunk_table, const int32_t* __restrict__ seg_counts,
    float* __restrict__ aux, float* __restrict__ prob_sum) {
  __shared__ int seg_start[kReduceMaxSegments + 1];
  __shared__ float red[kAuxThreads / 64];
  segment_starts(chunk_table, nchunks, segments, seg_start);
  float aux_part = 0.0f;
  for (int e = threadIdx.x; e < experts; e += kAuxThreads) {
    float total_p = 0.0f;
    int total_c = 0;
    for (int s = 0; s < segments; ++s) {
      const int c0 = seg_start[s];
      const float sp = c0 < seg_start[s + 1] ? part_p[(size_t)c0 * experts + e] : 0.0f;
      const int sc = seg_counts[(size_t)s * experts + e];
      total_p += sp;
      total_c += sc;
      if (mode == MI355X_ROUTE_SIGMOID_NOAUX_TC) {
        const int len = seg_offsets == nullptr ? tokens : seg_offsets[s + 1] - seg_offsets[s];
        const float freq = (float)sc * (float)experts / (float)(top_k * len);
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
  if (lane_id() == 0) red[threadIdx.x >> 6] = aux_part;
  __syncthreads();
  if (threadIdx.x == 0) {
    float total = 0.0f;
    for (int w = 0; w < kAuxThreads / 64; ++w) total += red[w];
    aux[0] = mode == MI355X_ROUTE_SIGMOID_NOAUX_TC ? total : (float)experts * total;
  }
}

template <int W, int PL>
__global__ void __launch_bounds__(256) router_bwd_kernel(
    const float* __restrict__ logits, const float* __restrict__ weights,
    const int32_t* __restrict__ ids, const float* __restrict__ dscore,
    const int32_t* __restrict__ slots, int tokens, int experts, int top_k, int mode,
    const float* __restrict__ grad_aux, const float* __restrict__ grad_ps,
    const int32_t* __restrict__ offsets, int segments, const int32_t* __restrict__ seg_offsets,
    const int32_t* __restrict__ seg_counts, float* __restrict__ grad_logits, uint16_t* __restrict__ pieces) {
  const int lane = threadIdx.x & (W - 1), gbase = lane_id() & ~(W - 1);
  const int token = blockIdx.x * (256 / W) + threadIdx.x / W;
  if (token >= tokens) return;
  constexpr int per_lane = PL;  // slots per lane (experts <= W * PL)
  const float* row = logits + (size_t)token * experts;
  float l[kMaxPerLane], g[kMaxPerLane];
  float gp[kMaxPerLane];  // grad_ps of the lane's experts (0 past `experts`)
  _Pragma("unroll") for (int i = 0; i < kMaxPerLane; ++i) {
    int e = lane + W * i;
    float x = -INFINITY, y = 0.0f;
    if (i < per_lane) {
      x = row[min(e, experts - 1)];
      if (grad_ps != nullptr) y = grad_ps[min(e, experts - 1)];
    }
    l[i] = (i < per_lane && e < experts) ? x : -INFINITY;
    gp[i] = (i < per_lane && e < experts) ? y : 0.0f;
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
      s[i] = (lane + W * i) < experts ? sigmoid_f(l[i]) : 0.0f;
      rs += s[i];
    }
    rs = group_sum<W>(rs);
    SLOTS(i) p[i] = s[i] / rs;
    // route_backward, sigmoid branch (moe_router.py:406-421).
    float sj = active ? sigmoid_f(row[idj]) : 0.0f;
    float score_sum = group_sum<W>(sj);
    float scaling = group_sum<W>(active ? wj : 0.0f);
    float dot = group_sum<W>(active ? gw * wj : 0.0f);
    float selg = active ? ((scaling * gw - dot) / score_sum) * sj * (1.0f - sj) : 0.0f;
    for (int j = 0; j < top_k; ++j) {
      float v = __shfl(selg, gbase + j, 64);
      int e = __shfl(idj, gbase + j, 64);
      SLOTS(i)
        if (e == lane + W * i) g[i] += v;
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
        int e = lane + W * i;
        const int cnt = seg_counts[(size_t)seg * experts + min(e, experts - 1)];
        f[i] = e < experts ? (float)cnt * (float)experts / (float)(top_k * len) : 0.0f;
        qf += p[i] * f[i];
      }
      qf = group_sum<W>(qf);
      float coef = grad_aux[0] / ((float)len * rs);
      SLOTS(i) g[i] += coef * (f[i] - qf) * s[i] * (1.0f - s[i]);
    }
    if (grad_ps != nullptr) {
      float pg = 0.0f;
      SLOTS(i) {
        int e = lane + W * i;
        pg += e < experts ? p[i] * gp[i] : 0.0f;
      }
      pg = group_sum<W>(pg);
      SLOTS(i) {
        int e = lane + W * i;
        if (e < experts) g[i] += (1.0f - s[i]) * p[i] * (gp[i] - pg);
      }
    }
  } else {
    float m = -INFINITY;
    SLOTS(i) m = fmaxf(m, l[i]);
    m = group_max<W>(m);
    float z = 0.0f;
    SLOTS(i) {
      p[i] = (lane + W * i) < experts ? __expf(l[i] - m) : 0.0f;
      z += p[i];
    }
    z = group_sum<W>(z);
    SLOTS(i) p[i] = p[i] / z;
    if (mode == MI355X_ROUTE_TOPK_THEN_SOFTMAX) {
      // p_sel (g - <g, p_sel>) scattered to the chosen experts.
      float dot = group_sum<W>(active ? gw * wj : 0.0f);
      float v = active ? wj * (gw - dot) : 0.0f;
      for (int j = 0; j < top_k; ++j) {
        float vj = __shfl(v, gbase + j, 64);
        int e = __shfl(idj, gbase + j, 64);
        SLOTS(i)
          if (e == lane + W * i) g[i] += vj;
      }
    } else {
      // -p * <g, p_sel> + scatter(g * p_sel).
      float psel = 0.0f;
      for (int j = 0; j < top_k; ++j) {
        int e = __shfl(idj, gbase + j, 64);
        float pe = 0.0f;
        SLOTS(i)
          if (e == lane + W * i) pe = p[i];
        pe = __shfl(pe, gbase + e % W, 64);
        if (lane == j) psel = pe;
      }
      float dot = group_sum<W>(active ? gw * psel : 0.0f);
      SLOTS(i) g[i] = -p[i] * dot;
      float v = active ? gw * psel : 0.0f;
      for (int j = 0; j < top_k; ++j) {
        float vj = __shfl(v, gbase + j, 64);
        int e = __shfl(idj, gbase + j, 64);
        SLOTS(i)
          if (e == lane + W * i) g[i] += vj;
      }
    }
    // Batch aux gradient (moe_router.py:455-473): c * p (f - <p, f>).
    if (grad_aux != nullptr) {
      float f[kMaxPerLane];
      float pf = 0.0f;
      SLOTS(i) {
        int e = lane + W * i;
        const int ec = min(e, experts - 1);
        const int cnt = offsets[ec + 1] - offsets[ec];
        f[i] = e < experts ? (float)cnt / (float)(tokens * top_k) : 0.0f;
        pf += p[i] * f[i];
      }
      pf = group_sum<W>(pf);
      float coef = grad_aux[0] * (float)experts / (float)tokens;
      SLOTS(i) g[i] += coef * p[i] * (f[i] - pf);
    }
    if (grad_ps != nullptr) {
      float pg = 0.0f;
      SLOTS(i) {
        int e = lane + W * i;
        pg += e < experts ? p[i] * gp[i] : 0.0f;
      }
      pg = group_sum<W>(pg);
      SLOTS(i) {
        int e = lane + W * i;
        if (e < experts) g[i] += p[i] * (gp[i] - pg);
      }
    }
  }
  if (grad_logits != nullptr) {
    float* out = grad_logits + (size_t)token * experts;
    SLOTS(i) {
      int e = lane + W * i;
      if (e < experts) out[e] = g[i];
    }
  }
  if (pieces != nullptr) {
    // The two bf16 pieces of the router weight gradient's operand, side by
    // side in a row of 2E: hi = bf16(g), mid = bf16(g - hi) (both rounded to
    // nearest even, as torch's casts).
    uint16_t* row_out = pieces + (size_t)token * 2 * experts;
    SLOTS(i) {
      int e = lane + W * i;
      if (e < experts) {
        const uint16_t hi = f32_to_bf16(g[i]);
        row_out[e] = hi;
        row_out[experts + e] = f32_to_bf16(g[i] - bf16_to_f32(hi));
      }
    }
  }
}

// Launch `kernel<W, PL>` for the token-group width and expert slots per lane
// that fit: W = 16 with PL in {1, 2, 4, 8} when experts <= 128 and top_k <= 16
// (and `narrow` allows it), else W = 64 with the smallest PL in {1, 2, 4, 8}
// covering ceil(experts / 64). Slots past `experts` are masked.
template <template <int, int> class K, typename Launch>
void launch_by_width(int experts, int top_k, bool narrow, Launch&& launch) {
  if (narrow && experts <= kRowExperts && top_k <= kRowTopK) {
    const int need = (experts + 15) / 16;
    if (need <= 1) launch(K<16, 1>::fn, 16);
    else if (need <= 2) launch(K<16, 2>::fn, 16);
    else if (need <= 4) launch(K<16, 4>::fn, 16);
    else launch(K<16, 8>::fn, 16);
    return;
  }
  const int need = (experts + 63) / 64;
  if (need <= 1) launch(K<64, 1>::fn, 64);
  else if (need <= 2) launch(K<64, 2>::fn, 64);
  else if (need <= 4) launch(K<64, 4>::fn, 64);
  else launch(K<64, 8>::fn, 64);
}
template <int W, int PL> struct TopkK { static constexpr auto fn = router_topk_kernel<W, PL>; };
template <int W, int PL> struct StatsK { static constexpr auto fn = router_stats_partial_kernel<W, PL>; };
template <int W, int PL> struct BwdK { static constexpr auto fn = router_bwd_kernel<W, PL>; };

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
  // Group-limited selection keeps a whole wavefront per token.
  const bool grouped = mode == MI355X_ROUTE_SIGMOID_NOAUX_TC && topk_group < n_group;
  launch_by_width<TopkK>(experts, top_k, !grouped, [&](auto kernel, int width) {
    const int per_block = 256 / width;
    hipLaunchKernelGGL(kernel, dim3((tokens + per_block - 1) / per_block), dim3(256), 0,
                       (hipStream_t)stream, logits, tokens, experts, top_k, mode, bias, n_group,
                       topk_group, routed_scaling, forced_ids, weights, ids);
  });
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
  launch_by_width<StatsK>(experts, top_k, true, [&](auto kernel, int) {
    hipLaunchKernelGGL(kernel, dim3(nchunks), dim3(256), 0, s, logits, ids, tokens, experts, top_k,
                       mode, seg_offsets, chunk_table, part_p, part_c);
  });
  MI355X_LAUNCH_CHECK();
  if (segments <= kReduceMaxSegments) {
    const long long pairs = (long long)segments * experts;
    const int per_block = 256 / kPairLanes;
    hipLaunchKernelGGL(router_stats_pairs_kernel, dim3((unsigned)((pairs + per_block - 1) / per_block)),
                       dim3(256), 0, s, part_p, part_c, nchunks, experts, segments, chunk_table,
                       seg_counts);
    MI355X_LAUNCH_CHECK();
    hipLaunchKernelGGL(router_stats_aux_kernel, dim3(1), dim3(kAuxThreads), 0, s, part_p, nchunks,
                       tokens, experts, top_k, mode, segments, seg_offsets, chunk_table,
                       seg_counts, aux, prob_sum);
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
  launch_by_width<BwdK>(experts, top_k, true, [&](auto kernel, int width) {
    const int per_block = 256 / width;
    hipLaunchKernelGGL(kernel, dim3((tokens + per_block - 1) / per_block), dim3(256), 0,
                       (hipStream_t)stream, logits, weights, ids, dscore, slots, tokens, experts,
                       top_k, mode, grad_aux, grad_prob_sum, offsets, segments, seg_offsets,
                       seg_counts, grad_logits, pieces);
  });
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
