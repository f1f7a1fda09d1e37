// Factor gradients of expert LoRA as grouped reductions over routed rows:
//
//   out[e][m][n] = sum over the rows j of expert e of big[j][m] * small[j][n]
//
// with big a bf16 routed-row matrix [rows, M] (dh or the scaled activation
// a'), small a bf16 rank-R matrix [rows, R] (z13 or u2; R a multiple of 16
// up to 64) and fp32 sums. Rows are expert-sorted (offsets[E+1]); nothing is
// read on the host, so the call does not synchronize.
//
// The work streams `big` once from HBM (R/16 times for R > 16). Each block
// takes a chunk of up to `chunk` rows of one expert and 2048 columns: a
// thread owns 8 consecutive columns and 16 rank sums for each (128 fp32
// accumulators), and walks the chunk's rows in order, reading its 16-byte
// slice of each row; the chunk's rank values sit in LDS as fp32 and every
// lane reads the same ones (broadcast). Partial sums of each chunk go to a
// workspace; a second kernel adds an expert's chunks in chunk order. Both
// orders are fixed, so the result is bitwise repeatable.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kCols = 8;                      // columns per thread
constexpr int kBlockCols = kThreads * kCols;  // 2048
constexpr int kRanks = 16;                    // rank sums per pass (blockIdx.z picks the 16)
constexpr int kStageRows = 256;               // rank rows staged in LDS at a time
constexpr int kMaxExperts = 1024;

// prefix[e] = number of chunks before expert e (chunks of `chunk` rows).
__device__ void chunk_prefix(const int32_t* __restrict__ offsets, int experts, int chunk,
                             int* prefix) {
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < experts; ++e) {
      prefix[e] = run;
      run += (offsets[e + 1] - offsets[e] + chunk - 1) / chunk;
    }
    prefix[experts] = run;
  }
  __syncthreads();
}

__device__ __forceinline__ int expert_of_chunk(const int* prefix, int experts, int c) {
  int lo = 0, hi = experts - 1;  // last e with prefix[e] <= c
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= c) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ void __launch_bounds__(kThreads) rank_grad_partial_kernel(
    const uint16_t* __restrict__ big, int M, const uint16_t* __restrict__ small, int R,
    const int32_t* __restrict__ offsets, int experts, int chunk, float* __restrict__ partial) {
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ float4 svals[kStageRows][kRanks / 4];
  chunk_prefix(offsets, experts, chunk, prefix);
  const int c = blockIdx.y;
  if (c >= prefix[experts]) return;  // uniform over the block
  const int e = expert_of_chunk(prefix, experts, c);
  const int row0 = offsets[e] + (c - prefix[e]) * chunk;
  const int row1 = min(row0 + chunk, offsets[e + 1]);
  const int n0 = blockIdx.z * kRanks;
  const int col = blockIdx.x * kBlockCols + threadIdx.x * kCols;
  const bool active = col < M;  // M is a multiple of 8

  float acc[kCols][kRanks];
#pragma unroll
  for (int i = 0; i < kCols; ++i)
#pragma unroll
    for (int n = 0; n < kRanks; ++n) acc[i][n] = 0.0f;

  for (int s0 = row0; s0 < row1; s0 += kStageRows) {
    const int s1 = min(s0 + kStageRows, row1);
    __syncthreads();  // the previous stage's rank values are consumed
    {
      const int j = s0 + threadIdx.x;
      float v[kRanks];
      if (j < s1) {
        const uint4* p = (const uint4*)(small + (size_t)j * R + n0);
        unpack_bf16x8(p[0], v);
        unpack_bf16x8(p[1], v + 8);
      } else {
#pragma unroll
        for (int n = 0; n < kRanks; ++n) v[n] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < kRanks / 4; ++q)
        svals[threadIdx.x][q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
    __syncthreads();
    if (!active) continue;
    const uint16_t* src = big + (size_t)s0 * M + col;
    // Rows in groups of 4 with the group's loads issued first.
    int j = s0;
    for (; j + 4 <= s1; j += 4) {
      uint4 raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[u] = *(const uint4*)(src + (size_t)(j - s0 + u) * M);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float b[kCols];
        unpack_bf16x8(raw[u], b);
        const int lj = j - s0 + u;
#pragma unroll
        for (int q = 0; q < kRanks / 4; ++q) {
          const float4 s = svals[lj][q];
#pragma unroll
          for (int i = 0; i < kCols; ++i) {
            acc[i][4 * q] = fmaf(b[i], s.x, acc[i][4 * q]);
            acc[i][4 * q + 1] = fmaf(b[i], s.y, acc[i][4 * q + 1]);
            acc[i][4 * q + 2] = fmaf(b[i], s.z, acc[i][4 * q + 2]);
            acc[i][4 * q + 3] = fmaf(b[i], s.w, acc[i][4 * q + 3]);
          }
        }
      }
    }
    for (; j < s1; ++j) {
      float b[kCols];
      unpack_bf16x8(*(const uint4*)(src + (size_t)(j - s0) * M), b);
      const int lj = j - s0;
#pragma unroll
      for (int q = 0; q < kRanks / 4; ++q) {
        const float4 s = svals[lj][q];
#pragma unroll
        for (int i = 0; i < kCols; ++i) {
          acc[i][4 * q] = fmaf(b[i], s.x, acc[i][4 * q]);
          acc[i][4 * q + 1] = fmaf(b[i], s.y, acc[i][4 * q + 1]);
          acc[i][4 * q + 2] = fmaf(b[i], s.z, acc[i][4 * q + 2]);
          acc[i][4 * q + 3] = fmaf(b[i], s.w, acc[i][4 * q + 3]);
        }
      }
    }
  }
  if (!active) return;
  // partial[c][m][n] (n fastest, R wide): 16 rank sums of a column are 64 bytes.
  float* dst = partial + ((size_t)c * M + col) * R + n0;
#pragma unroll
  for (int i = 0; i < kCols; ++i)
#pragma unroll
    for (int q = 0; q < kRanks / 4; ++q)
      *(float4*)(dst + (size_t)i * R + 4 * q) =
          make_float4(acc[i][4 * q], acc[i][4 * q + 1], acc[i][4 * q + 2], acc[i][4 * q + 3]);
}

// out[e] = sum of expert e's chunks in chunk order (zeros for an expert with
// no rows); `transposed` writes out[e] as [R][M] instead of [M][R].
__global__ void __launch_bounds__(kThreads) rank_grad_reduce_kernel(
    const float* __restrict__ partial, int M, int R, const int32_t* __restrict__ offsets,
    int experts, int chunk, int transposed, float* __restrict__ out) {
  __shared__ int prefix[kMaxExperts + 1];
  chunk_prefix(offsets, experts, chunk, prefix);
  const int e = blockIdx.y;
  const size_t per = (size_t)M * R;
  const size_t i = ((size_t)blockIdx.x * kThreads + threadIdx.x) * 4;  // R % 4 == 0
  if (i >= per) return;
  float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int c = prefix[e]; c < prefix[e + 1]; ++c) {
    const float4 v = *(const float4*)(partial + (size_t)c * per + i);
    sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
  }
  if (!transposed) {
    *(float4*)(out + (size_t)e * per + i) = sum;
  } else {
    const int m = (int)(i / R), n = (int)(i % R);
    float* o = out + (size_t)e * per;
    o[(size_t)n * M + m] = sum.x;
    o[(size_t)(n + 1) * M + m] = sum.y;
    o[(size_t)(n + 2) * M + m] = sum.z;
    o[(size_t)(n + 3) * M + m] = sum.w;
  }
}

size_t max_chunks(int rows, int experts, int chunk) {
  return (size_t)(rows + chunk - 1) / chunk + (size_t)experts;
}

}  // namespace

extern "C" size_t mi355x_rank_grad_workspace_size(int rows, int experts, int m, int rank,
                                                  int chunk) {
  if (rows < 0 || experts <= 0 || m <= 0 || rank <= 0 || chunk <= 0) return 0;
  return max_chunks(rows, experts, chunk) * (size_t)m * (size_t)rank * sizeof(float);
}

extern "C" int mi355x_rank_grad(const void* big, int rows, int m, const void* small, int rank,
                                const int32_t* offsets, int experts, int chunk, int transposed,
                                float* out, void* workspace, size_t workspace_bytes,
                                void* stream) {
  MI355X_REQUIRE(m > 0 && m % 8 == 0, "rank_grad: the wide dimension must be a multiple of 8");
  MI355X_REQUIRE(rank > 0 && rank % 16 == 0 && rank <= 64,
                 "rank_grad: the rank must be a multiple of 16 up to 64 (pad with zeros)");
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "rank_grad: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(chunk >= 1 && chunk <= (1 << 20), "rank_grad: bad chunk size %d", chunk);
  MI355X_REQUIRE(rows >= 0, "rank_grad: negative row count");
  MI355X_REQUIRE(workspace_bytes >= mi355x_rank_grad_workspace_size(rows, experts, m, rank, chunk),
                 "rank_grad: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const size_t chunks = max_chunks(rows, experts, chunk);
  MI355X_REQUIRE(chunks <= 65535, "rank_grad: %zu row chunks exceed the grid; raise the chunk",
                 chunks);
  float* partial = (float*)workspace;
  if (rows > 0) {
    const dim3 grid((m + kBlockCols - 1) / kBlockCols, (unsigned)chunks, rank / kRanks);
    hipLaunchKernelGGL(rank_grad_partial_kernel, grid, dim3(kThreads), 0, s,
                       (const uint16_t*)big, m, (const uint16_t*)small, rank, offsets, experts,
                       chunk, partial);
    MI355X_LAUNCH_CHECK();
  }
  const size_t per = (size_t)m * rank;
  const dim3 rgrid((unsigned)((per / 4 + kThreads - 1) / kThreads), experts);
  hipLaunchKernelGGL(rank_grad_reduce_kernel, rgrid, dim3(kThreads), 0, s, partial, m, rank,
                     offsets, experts, chunk, transposed, out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
