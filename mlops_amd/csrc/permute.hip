// Token permutation: the stable counting sort that groups routed rows by
// expert, the dispatch that quantizes each token once and writes its k routed
// copies, and the token-parallel combine / token-sum of the way back.
#include <mutex>

#include "common.h"

namespace {

constexpr int kPlanChunk = 1024;  // assignments per plan block
constexpr int kPlanThreads = 256;
constexpr int kMaxExperts = 1024;

// Pass 1: per-chunk expert histogram.
__global__ void __launch_bounds__(kPlanThreads) plan_hist_kernel(
    const int32_t* __restrict__ ids, int n, int experts, int32_t* __restrict__ hist) {
  __shared__ int h[kMaxExperts];
  for (int e = threadIdx.x; e < experts; e += blockDim.x) h[e] = 0;
  __syncthreads();
  const int start = blockIdx.x * kPlanChunk;
  const int end = min(n, start + kPlanChunk);
  for (int i = start + threadIdx.x; i < end; i += blockDim.x) atomicAdd(&h[ids[i]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += blockDim.x)
    hist[(size_t)blockIdx.x * experts + e] = h[e];
}

// Pass 2 (one block): expert totals, their exclusive scan (offsets), and each
// chunk's starting position per expert (written over the histogram). Each
// expert's chunks are split over G threads (G * experts <= the block), thread
// (part, e) taking a contiguous range of chunks; its counts are loaded in
// batches of sixteen before any is used, the parts' totals meet in LDS, and a
// second pass rewrites the range with the running positions.
__global__ void __launch_bounds__(kMaxExperts) plan_scan_kernel(
    int32_t* __restrict__ hist, int chunks, int experts, int n, int64_t* __restrict__ counts,
    int32_t* __restrict__ offsets) {
  __shared__ int scan[kMaxExperts];
  __shared__ int part_total[kMaxExperts];  // [part][expert]
  constexpr int kBatch = 16;
  const int tid = threadIdx.x;
  int parts = 1;
  while (parts * 2 * experts <= kMaxExperts) parts *= 2;
  const int e = tid % experts, part = tid / experts;
  const bool active = part < parts;
  const int per = (chunks + parts - 1) / parts;
  const int c_begin = min(chunks, part * per), c_end = min(chunks, c_begin + per);
  int local = 0;
  if (active) {
    for (int c0 = c_begin; c0 < c_end; c0 += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        v[j] = c0 + j < c_end ? hist[(size_t)(c0 + j) * experts + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) local += v[j];
    }
    part_total[part * experts + e] = local;
  }
  __syncthreads();
  // Expert totals and the parts' exclusive prefixes.
  int total = 0, before = 0;
  if (active) {
    for (int p = 0; p < parts; ++p) {
      const int t = part_total[p * experts + e];
      if (p < part) before += t;
      total += t;
    }
  }
  scan[tid] = (active && part == 0) ? total : 0;
  __syncthreads();
  for (int o = 1; o < kMaxExperts; o <<= 1) {
    int v = tid >= o ? scan[tid - o] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  // scan[e] is now the inclusive prefix of expert totals over experts 0..e
  if (active) {
    const int base = scan[e] - total;  // exclusive prefix
    if (part == 0) {
      counts[e] = total;
      offsets[e] = base;
    }
    int run = base + before;
    for (int c0 = c_begin; c0 < c_end; c0 += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        v[j] = c0 + j < c_end ? hist[(size_t)(c0 + j) * experts + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (c0 + j < c_end) hist[(size_t)(c0 + j) * experts + e] = run;
        run += v[j];
      }
    }
  }
  if (tid == 0) offsets[experts] = n;
}

// Pass 3: stable scatter. A chunk is walked in 256-element tiles in index
// order; inside a tile, equal ids are ranked by wave (ballot match on the
// id's bits) and by lane, so order is the stable argsort.
__global__ void __launch_bounds__(kPlanThreads) plan_scatter_kernel(
    const int32_t* __restrict__ ids, int n, int experts, const int32_t* __restrict__ base,
    int32_t* __restrict__ order, int32_t* __restrict__ slots) {
  __shared__ int running[kMaxExperts];
  __shared__ int wave_count[kPlanThreads / 64][kMaxExperts];
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    running[e] = base[(size_t)blockIdx.x * experts + e];
#pragma unroll
    for (int w = 0; w < kPlanThreads / 64; ++w) wave_count[w][e] = 0;
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6;
  int bits = 1;
  while ((1 << bits) < experts + 1) ++bits;
  const int start = blockIdx.x * kPlanChunk;
  const int end = min(n, start + kPlanChunk);
  for (int tile = start; tile < end; tile += kPlanThreads) {
    const int i = tile + threadIdx.x;
    const bool valid = i < end;
    const int e = valid ? ids[i] : experts;  // invalid lanes share a sentinel id
    uint64_t peers = __ballot(1);
    for (int b = 0; b < bits; ++b) {
      uint64_t ones = __ballot((e >> b) & 1);
      peers &= ((e >> b) & 1) ? ones : ~ones;
    }
    const int rank = __popcll(peers & lanes_below());
    const bool leader = rank == 0;
    const int cnt = __popcll(peers);
    if (valid && leader) wave_count[wave][e] = cnt;
    __syncthreads();
    if (valid) {
      int pos = running[e] + rank;
      for (int w = 0; w < wave; ++w) pos += wave_count[w][e];
      order[pos] = i;
      slots[i] = pos;
    }
    __syncthreads();
    if (valid && leader) {
      atomicAdd(&running[e], cnt);
      wave_count[wave][e] = 0;
    }
    __syncthreads();
  }
}

// Dispatch + 1x128 quantization: one wave per token; lane handles 8
// consecutive columns per 512-column step, 16 lanes make one 128 block.
__global__ void __launch_bounds__(256) permute_quantize_kernel(
    const uint16_t* __restrict__ x, int tokens, int width, int top_k,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ q, float* __restrict__ scales,
    int rows) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int t = blockIdx.x * 4 + wave;
  if (t >= tokens) return;
  int dest[32];
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < top_k) dest[j] = slots[(size_t)t * top_k + j];
  const uint16_t* src = x + (size_t)t * width;
  // 16 columns per lane (a 128-column scale group is 8 lanes), so each
  // destination row gets one 16-byte store per lane: a wave writes 1 KB of
  // whole lines per store. The row's loads (up to 2 chunks of 1024 columns)
  // are issued before any store: loads and stores share one completion
  // counter, so a load issued after a store would wait for it.
  constexpr int kRowChunks = 2;
  for (int base0 = 0; base0 < width; base0 += 1024 * kRowChunks) {
    uint4 raw[kRowChunks][2];
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c) {
      const int col = base0 + c * 1024 + lane * 16;
      raw[c][0] = raw[c][1] = make_uint4(0, 0, 0, 0);
      if (col < width) {
        raw[c][0] = load_stream(src + col);
        raw[c][1] = load_stream(src + col + 8);
      }
    }
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c) {
      const int col = base0 + c * 1024 + lane * 16;
      if (base0 + c * 1024 >= width) break;  // uniform over the wave
      float v[16];
      unpack_bf16x8(raw[c][0], v);
      unpack_bf16x8(raw[c][1], v + 8);
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
      amax = group_amax<8>(amax);
      const float s = fmaxf(amax * kInv448, kMinScale);
      const uint2 lo = quant8(v, s), hi = quant8(v + 8, s);
      const uint4 packed = make_uint4(lo.x, lo.y, hi.x, hi.y);
      if (col < width) {
        const int kb = col >> 7;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
          if (j < top_k) {
            store_stream(q + (size_t)dest[j] * width + col, packed);
            if ((lane & 7) == 0) scales[(size_t)kb * rows + dest[j]] = s;
          }
        }
      }
    }
  }
}

// out[t] = residual[t] + sum_j w[t,j] * y[slot[t,j]] (fp32, j order), one
// block per token, 8 columns per thread.
__global__ void __launch_bounds__(256) combine_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ slots,
    const float* __restrict__ weights, const uint16_t* __restrict__ residual, int top_k,
    int width, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  for (int col = threadIdx.x * 8; col < width; col += blockDim.x * 8) {
    float acc[8];
    if (residual != nullptr) {
      uint4 r = load_stream(residual + (size_t)t * width + col);
      uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = bf16_to_f32(w4[i] & 0xffff);
        acc[2 * i + 1] = bf16_to_f32(w4[i] >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    }
    for (int j = 0; j < top_k; ++j) {
      const size_t flat = (size_t)t * top_k + j;
      const int slot = slots[flat];
      const float w = weights != nullptr ? weights[flat] : 1.0f;
      uint4 r = load_stream(y + (size_t)slot * width + col);
      uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (weights != nullptr) {
          acc[2 * i] += bf16_to_f32(w4[i] & 0xffff) * w;
          acc[2 * i + 1] += bf16_to_f32(w4[i] >> 16) * w;
        } else {
          acc[2 * i] += bf16_to_f32(w4[i] & 0xffff);
          acc[2 * i + 1] += bf16_to_f32(w4[i] >> 16);
        }
      }
    }
    uint4 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    store_stream(out + (size_t)t * width + col, o);
  }
}

// ------------------------------------------------ allocation-free variant
// The plan's only scratch is the per-chunk histogram (chunks x experts int32).
// The allocation-free entry point keeps it in this file-scope device array, one
// copy per GPU, held until the process ends. The histogram pass writes every
// entry the later passes read, so nothing needs clearing between calls; calls
// that overlap on one GPU share the array and race.
constexpr size_t kPlanScratchInts = size_t(1) << 20;  // 4 MiB
__device__ __align__(256) int32_t scratch[kPlanScratchInts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's copy of `scratch`, looked up once per device
// with that device current. The array's name is only a host-side stand-in and
// is never passed to a kernel or a copy.
int plan_scratch(int32_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  MI355X_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices,
                 "permute_plan_noalloc: no current device (%s)", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    MI355X_REQUIRE(e == hipSuccess && p != nullptr,
                   "permute_plan_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = (int32_t*)p;
  }
  *out = g_scratch_ptr[dev];
  return MI355X_OK;
}

}  // namespace

extern "C" size_t mi355x_permute_plan_workspace_size(int assignments, int experts) {
  size_t chunks = ((size_t)assignments + kPlanChunk - 1) / kPlanChunk;
  return (chunks ? chunks : 1) * (size_t)experts * sizeof(int32_t) + 256;
}

extern "C" int mi355x_permute_plan(const int32_t* ids, int assignments, int experts,
                                   int64_t* counts, int32_t* offsets, int32_t* order,
                                   int32_t* slots, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "permute_plan: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(assignments >= 0, "permute_plan: negative assignments");
  MI355X_REQUIRE(workspace_bytes >= mi355x_permute_plan_workspace_size(assignments, experts),
                 "permute_plan: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const int chunks = (assignments + kPlanChunk - 1) / kPlanChunk;
  int32_t* hist = (int32_t*)workspace;
  if (chunks > 0) {
    hipLaunchKernelGGL(plan_hist_kernel, dim3(chunks), dim3(kPlanThreads), 0, s, ids,
                       assignments, experts, hist);
    MI355X_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(kMaxExperts), 0, s, hist, chunks, experts,
                     assignments, counts, offsets);
  MI355X_LAUNCH_CHECK();
  if (chunks > 0) {
    hipLaunchKernelGGL(plan_scatter_kernel, dim3(chunks), dim3(kPlanThreads), 0, s, ids,
                       assignments, experts, hist, order, slots);
    MI355X_LAUNCH_CHECK();
  }
  return MI355X_OK;
}

extern "C" size_t mi355x_permute_plan_noalloc_max_assignments(int experts) {
  if (experts <= 0 || experts > kMaxExperts) return 0;
  // the plan needs ceil(A / chunk) * experts ints plus 256 bytes of slack
  const size_t chunks = (kPlanScratchInts - 64) / (size_t)experts;
  return chunks * (size_t)kPlanChunk;
}

extern "C" int mi355x_permute_plan_noalloc(const int32_t* ids, int assignments, int experts,
                                           int64_t* counts, int32_t* offsets, int32_t* order,
                                           int32_t* slots, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts,
                 "permute_plan_noalloc: experts must be in [1, %d]", kMaxExperts);
  MI355X_REQUIRE(assignments >= 0, "permute_plan_noalloc: negative assignments");
  const size_t need = mi355x_permute_plan_workspace_size(assignments, experts);
  const size_t have = kPlanScratchInts * sizeof(int32_t);
  MI355X_REQUIRE(need <= have,
                 "permute_plan_noalloc: %d assignments x %d experts need %zu scratch bytes, "
                 "above the fixed %zu (at most %zu assignments at this expert count)",
                 assignments, experts, need, have,
                 mi355x_permute_plan_noalloc_max_assignments(experts));
  int32_t* hist = nullptr;
  const int rc = plan_scratch(&hist);
  if (rc != MI355X_OK) return rc;
  return mi355x_permute_plan(ids, assignments, experts, counts, offsets, order, slots, hist, have,
                             stream);
}

extern "C" int mi355x_permute_quantize_fp8(const void* x, int tokens, int width, int top_k,
                                           const int32_t* slots, uint8_t* q, float* scales,
                                           void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0, "permute_quantize: width must be a multiple of 128");
  MI355X_REQUIRE(top_k > 0 && top_k <= 32, "permute_quantize: top_k must be in [1, 32]");
  if (tokens == 0) return MI355X_OK;
  hipLaunchKernelGGL(permute_quantize_kernel, dim3((tokens + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x, tokens, width, top_k, slots, q,
                     scales, tokens * top_k);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_unpermute_combine(const void* y, const int32_t* slots, const float* weights,
                                        const void* residual, int tokens, int top_k, int width,
                                        void* out, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0, "combine: width must be a multiple of 8");
  MI355X_REQUIRE(weights != nullptr, "combine: route weights are required");
  if (tokens == 0) return MI355X_OK;
  hipLaunchKernelGGL(combine_kernel, dim3(tokens), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)y, slots, weights, (const uint16_t*)residual, top_k, width,
                     (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_unpermute_sum(const void* dx, const int32_t* slots, int tokens, int top_k,
                                    int width, void* out, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0, "unpermute_sum: width must be a multiple of 8");
  if (tokens == 0) return MI355X_OK;
  hipLaunchKernelGGL(combine_kernel, dim3(tokens), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)dx, slots, (const float*)nullptr, (const uint16_t*)nullptr,
                     top_k, width, (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
