// Thin grouped products of expert LoRA: out[r, 0:R] = sum_k a[r, k] bt[e][0:R, k]
// for the rows r of expert e (expert-sorted rows, offsets[E+1]). a is a
// bf16 routed-row matrix [rows, K] (dh or the activation), bt a bf16 factor
// [E, R, K] (K contiguous), R a multiple of 16 up to 64; fp32 sums, bf16 out.
//
// The products read all of `a` once and produce R columns, so they are
// bound by streaming `a` from HBM. One block takes 16 rows; its 4 waves
// split K four ways (v_mfma_f32_16x16x32_bf16: a lane holds 8 consecutive K
// values of its row or factor column), keep 4 K steps (8 at rank 16) of
// loads in flight, and meet in LDS. A 16-row block that spans an expert boundary is run once
// per expert present, storing only that expert's rows.
#include "common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
constexpr int kRankWaves = 4;
constexpr int kRankUnroll = 4;
constexpr int kMaxRank = 64;

__device__ __forceinline__ int expert_of(const int32_t* __restrict__ offsets, int experts,
                                         int row) {
  int lo = 0, hi = experts - 1;  // last e with offsets[e] <= row
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ void __launch_bounds__(64 * kRankWaves) rank_product_kernel(
    const uint16_t* __restrict__ a, int rows, int K, const uint16_t* __restrict__ bt, int R,
    const int32_t* __restrict__ offsets, int experts, uint16_t* __restrict__ out) {
  __shared__ float part[kRankWaves][16][kMaxRank + 1];
  const int row0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int lr = lane & 15, kq = 8 * (lane >> 4);
  const int row = min(row0 + lr, rows - 1);
  const int last = min(row0 + 15, rows - 1);
  const int e_lo = __builtin_amdgcn_readfirstlane(expert_of(offsets, experts, row0));
  const int e_hi = __builtin_amdgcn_readfirstlane(expert_of(offsets, experts, last));
  const int nc = R / 16;
  // This wave's K range, in 32-wide steps.
  const int steps = K / 32;
  const int s0 = steps * wave / kRankWaves, s1 = steps * (wave + 1) / kRankWaves;
  const uint16_t* arow = a + (size_t)row * K + kq;
  for (int e = e_lo; e <= e_hi; ++e) {
    if (offsets[e + 1] <= offsets[e]) continue;  // an empty expert inside the block's span
    v4f acc[kMaxRank / 16];
#pragma unroll
    for (int c = 0; c < kMaxRank / 16; ++c) acc[c] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* brow = bt + ((size_t)e * R + lr) * K + kq;
    int s = s0;
    if (nc == 1) {
      // Rank 16: every load of a group (8 K steps of the row and the factor)
      // issued before its MFMAs, so no MFMA waits on a single load.
      constexpr int kDeep = 2 * kRankUnroll;
      for (; s + kDeep <= s1; s += kDeep) {
        bf16x8_t af[kDeep], bf[kDeep];
#pragma unroll
        for (int u = 0; u < kDeep; ++u) af[u] = *(const bf16x8_t*)(arow + (s + u) * 32);
#pragma unroll
        for (int u = 0; u < kDeep; ++u) bf[u] = *(const bf16x8_t*)(brow + (s + u) * 32);
#pragma unroll
        for (int u = 0; u < kDeep; ++u)
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[u], bf[u], acc[0], 0, 0, 0);
      }
    }
    for (; s + kRankUnroll <= s1; s += kRankUnroll) {
      bf16x8_t af[kRankUnroll];
#pragma unroll
      for (int u = 0; u < kRankUnroll; ++u) af[u] = *(const bf16x8_t*)(arow + (s + u) * 32);
#pragma unroll
      for (int u = 0; u < kRankUnroll; ++u)
#pragma unroll
        for (int c = 0; c < kMaxRank / 16; ++c)
          if (c < nc) {
            const bf16x8_t bf = *(const bf16x8_t*)(brow + (size_t)c * 16 * K + (s + u) * 32);
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[u], bf, acc[c], 0, 0, 0);
          }
    }
    for (; s < s1; ++s) {
      const bf16x8_t af = *(const bf16x8_t*)(arow + s * 32);
#pragma unroll
      for (int c = 0; c < kMaxRank / 16; ++c)
        if (c < nc) {
          const bf16x8_t bf = *(const bf16x8_t*)(brow + (size_t)c * 16 * K + s * 32);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc[c], 0, 0, 0);
        }
    }
    // Output layout: acc[c][i] is row 4 * (lane / 16) + i, column c * 16 + lane % 16.
#pragma unroll
    for (int c = 0; c < kMaxRank / 16; ++c)
      if (c < nc)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][4 * (lane >> 4) + i][c * 16 + lr] = acc[c][i];
    __syncthreads();
    // Fixed-order sum over the waves, stored for this expert's rows.
    const int lo = max(offsets[e], row0), hi = min(offsets[e + 1], row0 + 16);
    for (int t = threadIdx.x; t < 16 * R; t += 64 * kRankWaves) {
      const int rr = t / R, col = t - rr * R;
      const int r = row0 + rr;
      if (r >= lo && r < hi) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kRankWaves; ++w) v += part[w][rr][col];
        out[(size_t)r * R + col] = f32_to_bf16(v);
      }
    }
    __syncthreads();  // part is reused by the next expert
  }
}

}  // namespace

extern "C" int mi355x_rank_product(const void* a, int rows, int k, const void* bt, int rank,
                                   const int32_t* offsets, int experts, void* out, void* stream) {
  MI355X_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "rank_product: K must be a multiple of 32");
  MI355X_REQUIRE(rank > 0 && rank % 16 == 0 && rank <= kMaxRank,
                 "rank_product: rank must be a multiple of 16 up to %d, got %d", kMaxRank, rank);
  MI355X_REQUIRE(experts > 0, "rank_product: experts must be positive");
  if (rows == 0) return MI355X_OK;
  hipLaunchKernelGGL(rank_product_kernel, dim3((rows + 15) / 16), dim3(64 * kRankWaves), 0,
                     (hipStream_t)stream, (const uint16_t*)a, rows, k, (const uint16_t*)bt, rank,
                     offsets, experts, (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
