// Router weight gradient on the bf16 MFMA: dW[e][h] = sum_t (hi[t][e] + mid[t][e]) x[t][h]
// with fp32 sums, where [hi | mid] are the bf16 pieces of the logit cotangent
// (hi = bf16(g), mid = bf16(g - hi)) that the router backward kernel writes
// side by side, token-major [T][2E], and x is the bf16 hidden state [T][H].
//
// Both operands run along the token (reduction) axis in memory, so the MFMA
// fragments, which want 8 consecutive tokens per lane, are read from row-
// major LDS tiles with ds_read_b64_tr_b16. Measured on MI355X: in each group
// of 16 lanes, lane j's element i is element j % 4 of the 4 that lane
// 4 i + j / 4 addressed. So if lane s of a group addresses token row
// k0 + s / 4 at column c0 + 4 (s % 4), lane j receives tokens k0 .. k0 + 3
// of column c0 + j; two such reads (k0 and k0 + 4) make the 8-token operand
// of v_mfma_f32_16x16x32_bf16.
//
// The hi and mid pieces multiply the same x tile into the same accumulators
// (two MFMAs per output tile and 32-token step). A workgroup owns a 128 x 256
// tile of dW over one token range, with its operand tiles copied by direct
// loads three steps ahead; the ranges' fp32 partials are summed in range
// order by a second kernel, so the result is deterministic.
#include "common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kRwM = 128;     // dW rows (experts) per workgroup
constexpr int kRwN = 256;     // dW columns (hidden) per workgroup
constexpr int kRwK = 32;      // tokens per step
constexpr int kRwRow = 512;   // bytes per staged row (256 bf16), unpadded
constexpr int kRwStages = 4;  // three steps' loads in flight while one is read
constexpr int kRwThreads = 512;
constexpr int kRwTile = kRwK * kRwRow;  // one operand's stage (16 KB)

__device__ __forceinline__ i16x4_t read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)p);
}

__device__ __forceinline__ bf16x8_t join(i16x4_t lo, i16x4_t hi) {
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  const i16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8_t, v);
}

// 16-byte unit u of staged row r sits at unit u ^ rsw(r). A fragment read
// takes rows 8g + 0..3 (and + 4) in each 16-lane group g, 32 bytes of each;
// the swizzle puts those 4 rows in 4 different 32-byte bank ranges, and
// groups 0 and 1 (read in the same cycle) in different halves.
__device__ __forceinline__ int rsw(int r) { return (2 * (r & 3)) | (8 * ((r >> 3) & 1)); }

// LDS byte address of a wave-uniform LDS pointer, as a scalar for M0.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr_t)p);
}
// global_load_lds_dwordx4: 64 lanes x 16 bytes into LDS at M0 + 16 * lane,
// from the wave-uniform base plus each lane's 32-bit byte offset. Issued as
// inline assembly, so the compiler does not count it: the kernel waits for
// these loads itself (wait_and_sync<N>).
__device__ __forceinline__ void dma16(const void* base, uint32_t off, const uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr(lds)), "v"(off), "s"(base) : "memory", "m0");
}
// Wait until at most N of this wave's loads are in flight, then barrier.
template <int N>
__device__ __forceinline__ void wait_and_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Stage layout: A rows = 128 hi columns then 128 mid columns of one token,
// B rows = 256 hidden columns of one token; 32 rows each, 512 bytes a row.
__global__ void __launch_bounds__(kRwThreads) router_wgrad_kernel(
    const uint16_t* __restrict__ pieces, const uint16_t* __restrict__ x, int tokens, int experts,
    int hidden, int range_tokens, int ranges, float* __restrict__ partial) {
  __shared__ __align__(1024) uint8_t smem[kRwStages * 2 * kRwTile];  // stages of (A tile, B tile)
  // Workgroup b runs on XCD b % 8. The n-tiles of one (expert tile, token
  // range) share that range's A rows: they are numbered so that they land on
  // one XCD, whose L2 then serves the A rows to all of them after one fetch.
  const int ntiles = hidden / kRwN, mtiles = (experts + kRwM - 1) / kRwM;
  const int b = blockIdx.x, per = ntiles * 8;
  const int group = b % 8 + 8 * (b / per);  // (expert tile, range) pair
  const int nt = (b / 8) % ntiles;
  if (group >= mtiles * ranges) return;  // padding of the last group
  const int mt = group % mtiles, range = group / mtiles;
  const int n0 = nt * kRwN, m0 = mt * kRwM;
  const int t_begin = range * range_tokens, t_end = min(tokens, t_begin + range_tokens);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  // Copies: a wave's direct load writes 1 KB = 2 staged rows; a step is 16
  // such loads per operand, 2 per wave. Lane L writes physical unit L % 32 of
  // row 2 i + L / 32 and so loads logical unit (L % 32) ^ rsw(row).
  const size_t a_row = (size_t)2 * experts * 2, b_row = (size_t)hidden * 2;
  uint32_t a_off[2], b_off[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 2 * (wave * 2 + j) + (lane >> 5);
    const int u = (lane & 31) ^ rsw(row);
    // A unit u: hi (u < 16) or mid columns m0 + 8 (u % 16), clamped into the
    // row (rows past `experts` are never stored).
    const int col = min(m0 + 8 * (u & 15), experts - 8);
    a_off[j] = (uint32_t)(row * a_row + 2 * ((u >> 4) * experts + col));
    b_off[j] = (uint32_t)(row * b_row + 2 * (n0 + 8 * u));
  }
  auto issue = [&](int step) {
    uint8_t* st = smem + (step % kRwStages) * 2 * kRwTile;
    const size_t t0 = (size_t)t_begin + (size_t)step * kRwK;
    const uint8_t* abase = (const uint8_t*)pieces + t0 * a_row;
    const uint8_t* bbase = (const uint8_t*)x + t0 * b_row;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rows0 = 2 * (wave * 2 + j);
      dma16(abase, a_off[j], st + rows0 * kRwRow);
      dma16(bbase, b_off[j], st + kRwTile + rows0 * kRwRow);
    }
  };

  // Wave tile: 64 experts (4 m-tiles) x 64 hidden columns (4 n-tiles).
  const int wm = (wave >> 2) * 64, wn = (wave & 3) * 64;
  const int g = lane >> 4, s = lane & 15;
  // Lane s of group g addresses token row 8g + s/4 (+4 for the second read),
  // column c0 + 4 (s % 4): 8 bytes at byte 2 c0 + 8 (s % 4) of the row.
  const int rd_row = 8 * g + (s >> 2);
  const int rsw0 = rsw(rd_row), rsw1 = rsw(rd_row + 4);
  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[i][q] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

  // 8 bytes at logical byte offset `byte` (a multiple of 8) of staged rows
  // rd_row and rd_row + 4.
  auto frag = [&](const uint8_t* tile, int byte) {
    const int u = byte >> 4, h = byte & 15;
    const uint8_t* p0 = tile + rd_row * kRwRow + 16 * (u ^ rsw0) + h;
    const uint8_t* p1 = tile + (rd_row + 4) * kRwRow + 16 * (u ^ rsw1) + h;
    return join(read_tr16(p0), read_tr16(p1));
  };
  auto compute = [&](const uint8_t* st) {
    const uint8_t* A = st;
    const uint8_t* B = st + kRwTile;
    bf16x8_t bf[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bf[q] = frag(B, 2 * (wn + 16 * q) + 8 * (s & 3));
#pragma unroll
    for (int p = 0; p < 2; ++p) {  // hi, then mid
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8_t af = frag(A, p * 256 + 2 * (wm + 16 * i) + 8 * (s & 3));
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[i][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[q], acc[i][q], 0, 0, 0);
      }
    }
  };

  // Whole 32-token steps through the direct-load pipeline.
  const int full = max(0, t_end - t_begin) / kRwK;
#pragma unroll
  for (int k = 0; k < kRwStages - 1; ++k)
    if (k < full) issue(k);
  for (int k = 0; k < full; ++k) {
    // Step k's 4 loads have landed once at most 4 x (younger steps issued)
    // are in flight; the barrier also retires every wave's reads of step k - 1,
    // whose stage step k + 3 then refills.
    const int younger = min(full - 1 - k, kRwStages - 2);
    if (younger >= 2) wait_and_sync<8>();
    else if (younger == 1) wait_and_sync<4>();
    else wait_and_sync<0>();
    if (k + kRwStages - 1 < full) issue(k + kRwStages - 1);
    compute(smem + (k % kRwStages) * 2 * kRwTile);
  }
  // A partial last step (the last range only): masked register loads.
  const int tail = t_begin + full * kRwK;
  if (tail < t_end) {
    __syncthreads();  // every wave is done with the stages
    uint8_t* st = smem;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int idx = q * kRwThreads + tid, row = idx >> 5, pu = idx & 31;
      const int u = pu ^ rsw(row);
      const int t = tail + row;
      const int col = m0 + 8 * (u & 15);
      uint4 va = make_uint4(0, 0, 0, 0), vb = make_uint4(0, 0, 0, 0);
      if (t < t_end) {
        if (col < experts)
          va = *(const uint4*)(pieces + (size_t)t * 2 * experts + (u >> 4) * experts + col);
        vb = *(const uint4*)(x + (size_t)t * hidden + n0 + 8 * u);
      }
      *(uint4*)(st + row * kRwRow + 16 * pu) = va;
      *(uint4*)(st + kRwTile + row * kRwRow + 16 * pu) = vb;
    }
    __syncthreads();
    compute(st);
  }
  // acc[i][q][r]: expert m0 + wm + 16 i + 4 g + r, column n0 + wn + 16 q + s.
  float* out = partial + (size_t)range * experts * hidden;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm + 16 * i + 4 * g + r;
      if (m < experts) {
#pragma unroll
        for (int q = 0; q < 4; ++q) out[(size_t)m * hidden + n0 + wn + 16 * q + s] = acc[i][q][r];
      }
    }
}

// dW = sum over ranges of the partials, in range order; four columns per thread.
__global__ void __launch_bounds__(256) router_wgrad_reduce_kernel(const float* __restrict__ partial,
                                                                  int ranges, size_t count,
                                                                  float* __restrict__ out) {
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= count) return;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  constexpr int kBatch = 8;  // partials loaded before they are added (in order)
  for (int r0 = 0; r0 < ranges; r0 += kBatch) {
    float4 v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      v[j] = r0 + j < ranges ? *(const float4*)(partial + (size_t)(r0 + j) * count + i)
                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      acc.x += v[j].x;
      acc.y += v[j].y;
      acc.z += v[j].z;
      acc.w += v[j].w;
    }
  }
  *(float4*)(out + i) = acc;
}

// Token ranges: about one workgroup per CU (more ranges would add partial
// traffic, 4 bytes x E x H each), each range a whole number of 32-token steps.
int wgrad_ranges(int tokens, int experts, int hidden) {
  const int tiles = (hidden / kRwN) * ((experts + kRwM - 1) / kRwM);
  int ranges = (256 + tiles - 1) / tiles;
  const int max_ranges = (tokens + kRwK - 1) / kRwK;
  return ranges < 1 ? 1 : ranges > max_ranges ? max_ranges : ranges;
}

int wgrad_range_tokens(int tokens, int ranges) {
  const int per = (tokens + ranges - 1) / ranges;
  return (per + kRwK - 1) / kRwK * kRwK;
}

}  // namespace

extern "C" size_t mi355x_router_weight_grad_workspace_size(int tokens, int experts, int hidden) {
  if (tokens <= 0 || experts <= 0 || hidden <= 0) return 0;
  return (size_t)wgrad_ranges(tokens, experts, hidden) * experts * hidden * sizeof(float);
}

extern "C" int mi355x_router_weight_grad(const void* pieces, const void* x, int tokens, int experts,
                                         int hidden, float* grad_weight, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  MI355X_REQUIRE(tokens >= 0 && experts > 0 && experts % 8 == 0,
                 "router_weight_grad: experts must be a positive multiple of 8");
  MI355X_REQUIRE(hidden > 0 && hidden % kRwN == 0,
                 "router_weight_grad: hidden must be a multiple of %d", kRwN);
  MI355X_REQUIRE((size_t)tokens * 2 * experts < (1ull << 40), "router_weight_grad: too large");
  hipStream_t st = (hipStream_t)stream;
  const size_t count = (size_t)experts * hidden;
  if (tokens == 0) {  // zero ranges: the reduction writes zeros
    hipLaunchKernelGGL(router_wgrad_reduce_kernel, dim3((unsigned)((count / 4 + 255) / 256)),
                       dim3(256), 0, st, nullptr, 0, count, grad_weight);
    MI355X_LAUNCH_CHECK();
    return MI355X_OK;
  }
  MI355X_REQUIRE(workspace_bytes >= mi355x_router_weight_grad_workspace_size(tokens, experts, hidden),
                 "router_weight_grad: workspace too small");
  const int ranges = wgrad_ranges(tokens, experts, hidden);
  const int range_tokens = wgrad_range_tokens(tokens, ranges);
  float* partial = (float*)workspace;
  // Pairs of (expert tile, range) in groups of 8, each group's n-tiles
  // interleaved so that a pair's n-tiles share an XCD; padded to whole groups.
  const int pairs = ((experts + kRwM - 1) / kRwM) * ranges;
  dim3 grid((unsigned)((pairs + 7) / 8 * 8 * (hidden / kRwN)));
  hipLaunchKernelGGL(router_wgrad_kernel, grid, dim3(kRwThreads), 0, st,
                     (const uint16_t*)pieces,
                     (const uint16_t*)x, tokens, experts, hidden, range_tokens, ranges, partial);
  MI355X_LAUNCH_CHECK();
  hipLaunchKernelGGL(router_wgrad_reduce_kernel, dim3((unsigned)((count / 4 + 255) / 256)),
                     dim3(256), 0, st, partial, ranges, count, grad_weight);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
