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
//
// That register-operand form loads in the MFMA operand layout: a 16-lane
// quarter-wave reads 16 rows x 16 bytes, so each load instruction touches
// 16 cache lines at half use, and every wave reloads the factor. For K a
// multiple of 128 the staged form below is used instead: rows and factor
// are copied to LDS with direct loads (16 lanes per 256-byte row slice, so
// whole lines), three stages deep, and each wave reads its MFMA fragments
// from there. With few row blocks (rows / 32 below ~4 per CU) the K chunks
// are also split over `splits` blocks per row block, each writing fp32
// partial sums that a second kernel adds in split order, so that enough
// blocks stream at once.
#include "gemm_pipe.h"

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

// Staged form: a block of 4 waves takes 64 rows, a wave 16 rows over all of
// K, in chunks of 128 K (256 bytes per row). A chunk's row slices and the
// factor's R slices go to LDS with direct loads; chunk c of a row r sits at
// 16-byte position c ^ (r % 16), so the 16 rows of a fragment read fall in
// distinct banks. R is a template parameter so that each wave's loads per
// stage, 4 + R / 16, is a compile-time count for the wait.
constexpr int kStWaves = 4;
constexpr int kStRows = 16 * kStWaves;
constexpr int kStSlice = 256;  // bytes of one row per K chunk
constexpr int kStStages = 3;

template <int R>
__global__ void __launch_bounds__(64 * kStWaves) rank_product_staged_kernel(
    const uint16_t* __restrict__ a, int rows, int K, const uint16_t* __restrict__ bt,
    const int32_t* __restrict__ offsets, int experts, uint16_t* __restrict__ out,
    float* __restrict__ partial) {
  constexpr int A_BYTES = kStRows * kStSlice;              // 8 KB
  constexpr int B_BYTES = R * kStSlice;                    // 4-16 KB
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_PER_WAVE = A_BYTES / 1024 / kStWaves, B_PER_WAVE = B_BYTES / 1024 / kStWaves;
  static_assert(A_PER_WAVE * kStWaves * 1024 == A_BYTES && B_PER_WAVE * kStWaves * 1024 == B_BYTES,
                "whole 1 KB copies per wave");
  constexpr int LOADS = A_PER_WAVE + B_PER_WAVE;           // direct loads per wave per stage
  __shared__ __align__(1024) uint8_t smem[kStStages * STAGE];
  const int row0 = blockIdx.x * kStRows;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
  const int last = min(row0 + kStRows - 1, rows - 1);
  const int e_lo = __builtin_amdgcn_readfirstlane(expert_of(offsets, experts, row0));
  const int e_hi = __builtin_amdgcn_readfirstlane(expert_of(offsets, experts, last));
  // This block's K chunks: split blockIdx.y of gridDim.y.
  const int nall = K / 128, splits = gridDim.y, sp = blockIdx.y;
  const int ch0 = (int)((long long)nall * sp / splits);
  const int nch = (int)((long long)nall * (sp + 1) / splits) - ch0;
  const uint32_t pitch = (uint32_t)K * 2u;
  // Slice position of this lane's 16 bytes and the 16-byte chunk it holds.
  const int pos = lane & 15;
  for (int e = e_lo; e <= e_hi; ++e) {
    if (offsets[e + 1] <= offsets[e]) continue;  // an empty expert inside the block's span
    const uint8_t* fbase = (const uint8_t*)(bt + (size_t)e * R * K);
    auto issue = [&](int ch, int st) {
      uint8_t* base = smem + st * STAGE;
      const uint8_t* ab = (const uint8_t*)a + (size_t)(ch0 + ch) * kStSlice;
      const uint8_t* bb = fbase + (size_t)(ch0 + ch) * kStSlice;
#pragma unroll
      for (int i = 0; i < A_PER_WAVE; ++i) {  // 4 rows per copy
        const int j = wave * A_PER_WAVE + i, r = j * 4 + (lane >> 4);
        const uint32_t src = (uint32_t)min(row0 + r, rows - 1) * pitch + 16u * (uint32_t)(pos ^ (r & 15));
        pipe::dma16(ab, src, base + j * 1024);
      }
#pragma unroll
      for (int i = 0; i < B_PER_WAVE; ++i) {
        const int j = wave * B_PER_WAVE + i, r = j * 4 + (lane >> 4);
        const uint32_t src = (uint32_t)r * pitch + 16u * (uint32_t)(pos ^ (r & 15));
        pipe::dma16(bb, src, base + A_BYTES + j * 1024);
      }
    };
    v4f acc[R / 16];
#pragma unroll
    for (int c = 0; c < R / 16; ++c) acc[c] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    issue(0, 0);
    if (nch > 1) issue(1, 1);
    for (int ch = 0; ch < nch; ++ch) {
      // This chunk's copies; the next chunk's may stay in flight.
      if (ch + 1 < nch) pipe::wait_and_sync<LOADS>();
      else pipe::wait_and_sync<0>();
      // Into the stage every wave finished reading before this barrier.
      if (ch + 2 < nch) issue(ch + 2, (ch + 2) % kStStages);
      const uint8_t* ta = smem + (ch % kStStages) * STAGE;
      const uint8_t* tb = ta + A_BYTES;
      const int ar = wave * 16 + (lane & 15);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int c = ks * 4 + (lane >> 4);  // this lane's 8 K values of the 32-K step
        const int at = (c ^ (lane & 15)) * 16;
        const bf16x8_t af = *(const bf16x8_t*)(ta + ar * kStSlice + at);
#pragma unroll
        for (int cb = 0; cb < R / 16; ++cb) {
          const bf16x8_t bf = *(const bf16x8_t*)(tb + (cb * 16 + (lane & 15)) * kStSlice + at);
          acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc[cb], 0, 0, 0);
        }
      }
    }
    // acc[cb][i] is row 4 * (lane / 16) + i of the wave's 16, column cb * 16 + lane % 16.
    const int lo = max(offsets[e], row0), hi = min(offsets[e + 1], row0 + kStRows);
#pragma unroll
    for (int cb = 0; cb < R / 16; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = row0 + wave * 16 + 4 * (lane >> 4) + i;
        if (r >= lo && r < hi) {
          const size_t o = (size_t)r * R + cb * 16 + (lane & 15);
          if (partial == nullptr) out[o] = f32_to_bf16(acc[cb][i]);
          else partial[(size_t)sp * rows * R + o] = acc[cb][i];
        }
      }
    __syncthreads();  // the stages are refilled for the next expert
  }
}

// out = bf16(sum over splits of the partial sums, in split order).
__global__ void __launch_bounds__(256) rank_product_reduce_kernel(const float* __restrict__ partial,
                                                                  size_t n, int splits,
                                                                  uint16_t* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = partial[i];
  for (int p = 1; p < splits; ++p) s += partial[(size_t)p * n + i];
  out[i] = f32_to_bf16(s);
}

}  // namespace

extern "C" size_t mi355x_rank_product_workspace_size(int rows, int rank, int splits) {
  if (rows <= 0 || rank <= 0 || splits <= 1) return 0;
  return (size_t)splits * rows * rank * sizeof(float);
}

extern "C" int mi355x_rank_product(const void* a, int rows, int k, const void* bt, int rank,
                                   const int32_t* offsets, int experts, void* out, void* stream) {
  MI355X_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "rank_product: K must be a multiple of 32");
  MI355X_REQUIRE(rank > 0 && rank % 16 == 0 && rank <= kMaxRank,
                 "rank_product: rank must be a multiple of 16 up to %d, got %d", kMaxRank, rank);
  MI355X_REQUIRE(experts > 0, "rank_product: experts must be positive");
  if (rows == 0) return MI355X_OK;
  // The staged form: K in 128-wide chunks, and per-lane 32-bit byte offsets
  // into the rows and the factor.
  if (k % 128 == 0 && (uint64_t)rows * (uint64_t)k * 2u < (1ull << 32) &&
      (uint64_t)rank * (uint64_t)k * 2u < (1ull << 32)) {
    const dim3 grid((rows + kStRows - 1) / kStRows);
    auto launch = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, dim3(64 * kStWaves), 0, (hipStream_t)stream, (const uint16_t*)a, rows,
                         k, (const uint16_t*)bt, offsets, experts, (uint16_t*)out,
                         (float*)nullptr);
    };
    switch (rank) {
      case 16: launch(rank_product_staged_kernel<16>); break;
      case 32: launch(rank_product_staged_kernel<32>); break;
      case 48: launch(rank_product_staged_kernel<48>); break;
      default: launch(rank_product_staged_kernel<64>); break;
    }
    MI355X_LAUNCH_CHECK();
    return MI355X_OK;
  }
  hipLaunchKernelGGL(rank_product_kernel, dim3((rows + 15) / 16), dim3(64 * kRankWaves), 0,
                     (hipStream_t)stream, (const uint16_t*)a, rows, k, (const uint16_t*)bt, rank,
                     offsets, experts, (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_rank_product_split(const void* a, int rows, int k, const void* bt, int rank,
                                         const int32_t* offsets, int experts, int splits,
                                         void* out, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  MI355X_REQUIRE(splits >= 1 && splits <= 64, "rank_product_split: splits must be in [1, 64]");
  if (splits == 1) return mi355x_rank_product(a, rows, k, bt, rank, offsets, experts, out, stream);
  MI355X_REQUIRE(rows >= 0 && k > 0 && k % 128 == 0,
                 "rank_product_split: K must be a multiple of 128");
  MI355X_REQUIRE(rank > 0 && rank % 16 == 0 && rank <= kMaxRank,
                 "rank_product_split: rank must be a multiple of 16 up to %d, got %d", kMaxRank,
                 rank);
  MI355X_REQUIRE(splits <= k / 128, "rank_product_split: more splits than 128-wide K chunks");
  MI355X_REQUIRE(experts > 0, "rank_product_split: experts must be positive");
  MI355X_REQUIRE((uint64_t)rows * (uint64_t)k * 2u < (1ull << 32) &&
                     (uint64_t)rank * (uint64_t)k * 2u < (1ull << 32),
                 "rank_product_split: operands beyond 32-bit byte offsets");
  MI355X_REQUIRE(workspace_bytes >= mi355x_rank_product_workspace_size(rows, rank, splits),
                 "rank_product_split: workspace too small");
  if (rows == 0) return MI355X_OK;
  float* partial = (float*)workspace;
  const dim3 grid((rows + kStRows - 1) / kStRows, splits);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(64 * kStWaves), 0, (hipStream_t)stream, (const uint16_t*)a, rows, k,
                       (const uint16_t*)bt, offsets, experts, (uint16_t*)nullptr, partial);
  };
  switch (rank) {
    case 16: launch(rank_product_staged_kernel<16>); break;
    case 32: launch(rank_product_staged_kernel<32>); break;
    case 48: launch(rank_product_staged_kernel<48>); break;
    default: launch(rank_product_staged_kernel<64>); break;
  }
  MI355X_LAUNCH_CHECK();
  const size_t n = (size_t)rows * rank;
  hipLaunchKernelGGL(rank_product_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, partial, n, splits, (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
