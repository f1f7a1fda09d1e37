// Factor gradients of expert LoRA as grouped reductions over routed rows:
//
//   out[e][m][n] = sum over the rows j of expert e of big[j][m] * small[j][n]
//
// with big a bf16 routed-row matrix [rows, M] (dh or the scaled activation
// a'), small a bf16 rank-R matrix [rows, R] (z13 or u2; R a multiple of 16
// up to 64) and fp32 sums. Rows are expert-sorted (offsets[E+1]); nothing is
// read on the host, so the call does not synchronize.
//
// The work streams `big` once from HBM (R/16 times for R > 16), so it must
// run at HBM speed: with 16 ranks it is 16 FMAs per element read, which the
// VALU alone cannot keep up with, so the products run on the bf16 MFMA
// (v_mfma_f32_16x16x32_bf16: 16 columns x 16 ranks over 32 rows). Each block
// takes a chunk of up to `chunk` rows of one expert and 256 columns, 64 per
// wave, and walks the chunk 64 rows at a time through LDS. Partial sums of
// each chunk go to a workspace; a second kernel adds an expert's chunks in
// chunk order. Both orders are fixed, so the result is bitwise repeatable.
//
// Gathered form: row j of `big` may be a token row, big[gather[j] / div]
// (the routed row's token), and row j of `small` may be scaled by
// weight[index[j]] * alpha (index null: weight[j]), rounded to bf16 once as
// bf16(z * (w * alpha)): the token-side factor gradients of expert LoRA as
// reductions over each expert's routed rows, with no [tokens, E * R]
// scatter, and the route weight applied to a thin operand instead of a wide
// one.
#include "common.h"

namespace {

constexpr int kThreads = 256;                 // 4 waves
constexpr int kBlockColsMfma = 256;          // big columns per block, 64 per wave
constexpr int kRanks = 16;                    // rank sums per pass (blockIdx.z picks the 16)
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

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));

// A stage: 64 rows x 256 columns of big (32 KB) and 64 rows x 16 ranks of
// small, copied row-major into LDS with coalesced 16-byte loads. An MFMA
// operand needs 8 consecutive rows of one column per lane (the reduction runs
// over rows), so each fragment is gathered with eight 2-byte LDS reads; the
// row pitches put the four 8-row groups of a fragment read in different banks.
constexpr int kStRows = 64;
constexpr int kBigPitch = 2 * kBlockColsMfma + 8;   // bytes per staged big row (520)
constexpr int kSmallPitch = 2 * kRanks + 8;         // bytes per staged rank row (40)

__device__ __forceinline__ bf16x8_t gather8(const uint8_t* base, int pitch) {
  u16x8_t v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = *(const uint16_t*)(base + i * pitch);
  return __builtin_bit_cast(bf16x8_t, v);
}

__global__ void __launch_bounds__(kThreads) rank_grad_partial_kernel(
    const uint16_t* __restrict__ big, int M, const uint16_t* __restrict__ small, int R,
    const int32_t* __restrict__ offsets, int experts, int chunk, const int32_t* __restrict__ gather,
    int gather_div, const float* __restrict__ weight, const int32_t* __restrict__ windex,
    float alpha, float* __restrict__ partial) {
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ __align__(16) uint8_t big_s[kStRows * kBigPitch];
  __shared__ __align__(16) uint8_t small_s[kStRows * kSmallPitch];
  chunk_prefix(offsets, experts, chunk, prefix);
  const int c = blockIdx.y;
  if (c >= prefix[experts]) return;  // uniform over the block
  const int e = expert_of_chunk(prefix, experts, c);
  const int row0 = offsets[e] + (c - prefix[e]) * chunk;
  const int row1 = min(row0 + chunk, offsets[e + 1]);
  const int n0 = blockIdx.z * kRanks;
  const int m0 = blockIdx.x * kBlockColsMfma;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lcol = (tid & 31) * 8;  // this thread's 8 columns of the copy
  const bool col_ok = m0 + lcol < M;  // M is a multiple of 8

  v4f acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

  for (int s0 = row0; s0 < row1; s0 += kStRows) {
    // Loads first (rows past the chunk read as zeros), then the LDS stores;
    // the gather indices before the rows they select.
    int brow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(s0 + i * 8 + (tid >> 5), row1 - 1);
      brow[i] = gather != nullptr ? gather[r] / gather_div : r;
    }
    uint4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = s0 + i * 8 + (tid >> 5);
      v[i] = (r < row1 && col_ok) ? load_stream(big + (size_t)brow[i] * M + m0 + lcol)
                                  : make_uint4(0, 0, 0, 0);
    }
    uint4 sv = make_uint4(0, 0, 0, 0);
    if (tid < 2 * kStRows) {
      const int r = s0 + (tid >> 1);
      if (r < row1) {
        sv = *(const uint4*)(small + (size_t)r * R + n0 + (tid & 1) * 8);
        if (weight != nullptr) {
          const float f = weight[windex != nullptr ? windex[r] : r] * alpha;
          float z[8];
          unpack_bf16x8(sv, z);
          sv = make_uint4(pack_bf16x2(z[0] * f, z[1] * f), pack_bf16x2(z[2] * f, z[3] * f),
                          pack_bf16x2(z[4] * f, z[5] * f), pack_bf16x2(z[6] * f, z[7] * f));
        }
      }
    }
    __syncthreads();  // the previous stage's fragments are read
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint8_t* d = big_s + (i * 8 + (tid >> 5)) * kBigPitch + 2 * lcol;
      *(uint2*)d = make_uint2(v[i].x, v[i].y);
      *(uint2*)(d + 8) = make_uint2(v[i].z, v[i].w);
    }
    if (tid < 2 * kStRows) {
      uint8_t* d = small_s + (tid >> 1) * kSmallPitch + (tid & 1) * 16;
      *(uint2*)d = make_uint2(sv.x, sv.y);
      *(uint2*)(d + 8) = make_uint2(sv.z, sv.w);
    }
    __syncthreads();
    // D[m][n] += sum over 32 rows of big[row][m] * small[row][n], twice.
    const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int kk = 0; kk < kStRows; kk += 32) {
      const int rr = kk + 8 * g;
      const bf16x8_t b = gather8(small_s + rr * kSmallPitch + 2 * l16, kSmallPitch);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int m = wave * 64 + mb * 16 + l16;
        const bf16x8_t a = gather8(big_s + rr * kBigPitch + 2 * m, kBigPitch);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[mb], 0, 0, 0);
      }
    }
  }
  // acc[mb][i]: column m = m0 + wave * 64 + mb * 16 + 4 * (lane / 16) + i,
  // rank n = n0 + lane % 16. partial[c][m][n], R wide.
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + wave * 64 + mb * 16 + 4 * (lane >> 4) + i;
      if (m < M) partial[((size_t)c * M + m) * R + n0 + (lane & 15)] = acc[mb][i];
    }
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

namespace {
int rank_grad_launch(const void* big, int rows, int m, const void* small, int rank,
                     const int32_t* offsets, int experts, int chunk, const int32_t* gather,
                     int gather_div, const float* weight, const int32_t* windex, float alpha,
                     int transposed, float* out, void* workspace, size_t workspace_bytes,
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
    const dim3 grid((m + kBlockColsMfma - 1) / kBlockColsMfma, (unsigned)chunks, rank / kRanks);
    hipLaunchKernelGGL(rank_grad_partial_kernel, grid, dim3(kThreads), 0, s,
                       (const uint16_t*)big, m, (const uint16_t*)small, rank, offsets, experts,
                       chunk, gather, gather_div, weight, windex, alpha, partial);
    MI355X_LAUNCH_CHECK();
  }
  const size_t per = (size_t)m * rank;
  const dim3 rgrid((unsigned)((per / 4 + kThreads - 1) / kThreads), experts);
  hipLaunchKernelGGL(rank_grad_reduce_kernel, rgrid, dim3(kThreads), 0, s, partial, m, rank,
                     offsets, experts, chunk, transposed, out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
}  // namespace

extern "C" int mi355x_rank_grad(const void* big, int rows, int m, const void* small, int rank,
                                const int32_t* offsets, int experts, int chunk, int transposed,
                                float* out, void* workspace, size_t workspace_bytes,
                                void* stream) {
  return rank_grad_launch(big, rows, m, small, rank, offsets, experts, chunk, nullptr, 1, nullptr,
                          nullptr, 1.0f, transposed, out, workspace, workspace_bytes, stream);
}

extern "C" int mi355x_rank_grad_gather(const void* big, int big_rows, int m, const void* small,
                                       int rows, int rank, const int32_t* offsets, int experts,
                                       int chunk, const int32_t* gather, int gather_div,
                                       const float* weight, const int32_t* weight_index,
                                       float alpha, int transposed, float* out, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  MI355X_REQUIRE(gather_div >= 1, "rank_grad_gather: the gather divisor must be >= 1");
  MI355X_REQUIRE(gather != nullptr || big_rows == rows,
                 "rank_grad_gather: without a gather index big has the routed rows");
  MI355X_REQUIRE(big_rows >= 0, "rank_grad_gather: negative token count");
  return rank_grad_launch(big, rows, m, small, rank, offsets, experts, chunk, gather, gather_div,
                          weight, weight_index, alpha, transposed, out, workspace,
                          workspace_bytes, stream);
}
