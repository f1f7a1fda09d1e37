// Ragged grouped block-FP8 GEMMs for gfx950 (CDNA4).
//
// Math: every 128-wide K step is exactly one scale block of both operands,
// and one v_mfma_f32_16x16x128_f8f6f4 covers 16x16 outputs over those 128 K.
// So each MFMA produces the raw partial of one scale block, which is folded
// into the fp32 accumulator with its (row scale x weight-block scale):
//     acc += mfma(a, b, 0) * (sa[row] * sb)
// That is the reference's promoted accumulation (acc_sum += acc * scale per
// K block) at the granularity the hardware gives for free.
//
// MFMA operand layout (verified on MI355X): lane l supplies row l%16 of A
// and column l%16 of B, each as 32 consecutive K bytes starting at
// 32*(l/16); the 4 outputs of lane l are rows 4*(l/16)+i, column l%16.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid, workgroup tile 128x128,
// wave tile 64x64 (4x4 MFMA blocks). A and B tiles are staged through LDS
// (double buffered, 144-byte row pitch against bank conflicts) with 16-byte
// global loads. Workgroups are persistent: each computes the per-expert tile
// prefix from `offsets` once, then walks tiles blockIdx.x, +gridDim.x, ...
#include "common.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int PITCH = BK + 16;              // LDS bytes per staged row
constexpr int TILE_BYTES = BM * PITCH;      // one operand tile
constexpr int kThreads = 256;
constexpr int kMaxExperts = 512;

struct Lds {
  uint8_t a[2][TILE_BYTES];
  uint8_t b[2][TILE_BYTES];
  float sa[2][BM];
  float sb[2][BN];
};

// Exclusive prefix of ceil(rows_e / 128) over experts -> prefix[0..E].
__device__ void tile_prefix(const int32_t* __restrict__ offsets, int experts, int* prefix,
                            int* tmp) {
  const int t = threadIdx.x;
  const int per = (experts + kThreads - 1) / kThreads;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    int e = t * per + i;
    if (e < experts) local += (offsets[e + 1] - offsets[e] + BM - 1) / BM;
  }
  tmp[t] = local;
  __syncthreads();
  for (int o = 1; o < kThreads; o <<= 1) {
    int v = t >= o ? tmp[t - o] : 0;
    __syncthreads();
    tmp[t] += v;
    __syncthreads();
  }
  int run = tmp[t] - local;
  for (int i = 0; i < per; ++i) {
    int e = t * per + i;
    if (e < experts) {
      prefix[e] = run;
      run += (offsets[e + 1] - offsets[e] + BM - 1) / BM;
    }
  }
  if (t == kThreads - 1) prefix[experts] = tmp[t];
  __syncthreads();
}

__device__ __forceinline__ int find_expert(const int* prefix, int experts, int tile) {
  int lo = 0, hi = experts - 1;
  while (lo < hi) {  // last e with prefix[e] <= tile (skips empty experts)
    int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* tile, int row, int lane) {
  const uint8_t* p = tile + row * PITCH + 32 * (lane >> 4);
  uint4 x = *(const uint4*)p;
  uint4 y = *(const uint4*)(p + 16);
  v8i r;
  r[0] = x.x; r[1] = x.y; r[2] = x.z; r[3] = x.w;
  r[4] = y.x; r[5] = y.y; r[6] = y.z; r[7] = y.w;
  return r;
}

__device__ __forceinline__ v4f mfma_f8(v8i a, v8i b) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// One 128-K step of a 64x64 wave tile from the staged tiles.
__device__ __forceinline__ void wave_step(const uint8_t* ta, const uint8_t* tb, const float* sa,
                                          float sb, int wm, int wn, int lane, v4f (&acc)[4][4]) {
  v8i af[4], bf[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) af[i] = lds_frag(ta, wm * 64 + i * 16 + (lane & 15), lane);
#pragma unroll
  for (int j = 0; j < 4; ++j) bf[j] = lds_frag(tb, wn * 64 + j * 16 + (lane & 15), lane);
  float rs[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float4 s4 = *(const float4*)&sa[wm * 64 + i * 16 + 4 * (lane >> 4)];
    rs[i][0] = s4.x * sb; rs[i][1] = s4.y * sb; rs[i][2] = s4.z * sb; rs[i][3] = s4.w * sb;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v4f p = mfma_f8(af[i], bf[j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(p[r], rs[i][r], acc[i][j][r]);
    }
  }
}

// ---------------------------------------------------------------------------
// Forward / input-gradient GEMM over expert-sorted rows.
__global__ void __launch_bounds__(kThreads, 2) grouped_gemm_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ a_scale, int rows,
    const uint8_t* __restrict__ w, const float* __restrict__ w_scale, int w_scale_t, int experts,
    int N, int K, const int32_t* __restrict__ offsets, int interleave,
    const uint16_t* __restrict__ addend, uint16_t* __restrict__ out) {
  __shared__ __align__(16) Lds lds;
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ int tmp[kThreads];
  tile_prefix(offsets, experts, prefix, tmp);
  const int total_m_tiles = prefix[experts];
  const int n_tiles = N / BN;
  const int total = total_m_tiles * n_tiles;
  const int nk = K / BK;
  const int kb_count_w = K / 128, nb_count_w = N / 128;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int half_n = N / 2;

  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const int mt = tile / n_tiles, nt = tile % n_tiles;
    const int e = find_expert(prefix, experts, mt);
    const int row0 = offsets[e] + (mt - prefix[e]) * BM;
    const int nvalid = min(BM, offsets[e + 1] - row0);
    // B rows of this tile: 128 consecutive weight rows, or (interleave) 64
    // gate rows j0.. and 64 up rows half_n + j0.. of a gate/up weight.
    const int j0 = nt * 64;
    const uint8_t* wexp = w + (size_t)e * N * K;

    // Per-thread global load slots: 4 rows x 16 bytes of A and of B.
    const int lr = tid >> 3, lc = (tid & 7) * 16;
    const uint8_t* ga[4];
    const uint8_t* gb[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      int r = lr + 32 * p;
      int src = min(row0 + r, rows - 1);
      ga[p] = a + (size_t)src * K + lc;
      int wr = interleave ? (r < 64 ? j0 + r : half_n + j0 + (r - 64)) : nt * BN + r;
      gb[p] = wexp + (size_t)wr * K + lc;
    }
    // Weight-block scale row/col of each wave's columns for this tile.
    const int nb_mine = interleave ? (wn == 0 ? j0 / 128 : (half_n + j0) / 128) : nt;

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    uint4 ra[4], rb[4];
    float rsa = 0.0f, rsb = 0.0f;
    auto fetch = [&](int kb) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        ra[p] = *(const uint4*)(ga[p] + (size_t)kb * BK);
        rb[p] = *(const uint4*)(gb[p] + (size_t)kb * BK);
      }
      if (tid < BM) rsa = a_scale[(size_t)kb * rows + min(row0 + tid, rows - 1)];
      if (tid >= BM && tid < BM + 2) {
        int which = tid - BM;  // 0: first half of the tile's columns, 1: second
        int nb = interleave ? (which == 0 ? j0 / 128 : (half_n + j0) / 128) : nt;
        rsb = w_scale_t ? w_scale[((size_t)e * kb_count_w + kb) * nb_count_w + nb]
                        : w_scale[((size_t)e * nb_count_w + nb) * kb_count_w + kb];
      }
    };
    auto stash = [&](int buf) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        *(uint4*)&lds.a[buf][(lr + 32 * p) * PITCH + lc] = ra[p];
        *(uint4*)&lds.b[buf][(lr + 32 * p) * PITCH + lc] = rb[p];
      }
      if (tid < BM) lds.sa[buf][tid] = rsa;
      if (tid >= BM && tid < BM + 2) lds.sb[buf][tid - BM] = rsb;
    };

    fetch(0);
    stash(0);
    __syncthreads();
    for (int kb = 0; kb < nk; ++kb) {
      const int buf = kb & 1;
      if (kb + 1 < nk) fetch(kb + 1);
      const float sb = lds.sb[buf][interleave ? wn : 0];
      wave_step(lds.a[buf], lds.b[buf], lds.sa[buf], sb, wm, wn, lane, acc);
      if (kb + 1 < nk) stash(buf ^ 1);
      __syncthreads();
    }
    (void)nb_mine;

    // Epilogue: stage fp32 tile in LDS (over the operand buffers), then
    // write rows with 16-byte stores (+ addend), rounding once to bf16.
    float* stage = (float*)&lds;  // 128 x 128 fp32 = 64 KB
    constexpr int SP = BN + 4;    // staged row pitch in floats
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = wn * 64 + j * 16 + (lane & 15);
        const int oc = interleave ? (c < 64 ? 2 * c : 2 * (c - 64) + 1) : c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * 64 + i * 16 + 4 * (lane >> 4) + r;
          stage[row * SP + oc] = acc[i][j][r];
        }
      }
    }
    __syncthreads();
    const int col0 = nt * BN;  // interleaved output columns 2*j0.. = nt*128 too
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int idx = p * kThreads + tid;  // 2048 chunks of 8 columns
      const int r = idx >> 4, c8 = (idx & 15) * 8;
      if (r < nvalid) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = stage[r * SP + c8 + i];
        const size_t off = (size_t)(row0 + r) * N + col0 + c8;
        if (addend != nullptr) {
          uint4 c = *(const uint4*)(addend + off);
          uint32_t w4[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[2 * i] += bf16_to_f32(w4[i] & 0xffff);
            v[2 * i + 1] += bf16_to_f32(w4[i] >> 16);
          }
        }
        uint4 o;
        o.x = pack_bf16x2(v[0], v[1]);
        o.y = pack_bf16x2(v[2], v[3]);
        o.z = pack_bf16x2(v[4], v[5]);
        o.w = pack_bf16x2(v[6], v[7]);
        *(uint4*)(out + off) = o;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Weight-gradient GEMM: out[e][m][n] = sum over expert e's padded row blocks
// of p[m][row] * q[n][row] with per-(feature, block) scales on both sides.
__global__ void __launch_bounds__(kThreads, 2) wgrad_gemm_kernel(
    const uint8_t* __restrict__ p, const float* __restrict__ p_scale, int Mf,
    const uint8_t* __restrict__ q, const float* __restrict__ q_scale, int Nf, int padded,
    const int32_t* __restrict__ offsets, int experts, void* __restrict__ out, int out_fp32) {
  __shared__ __align__(16) Lds lds;
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ int tmp[kThreads];
  tile_prefix(offsets, experts, prefix, tmp);
  const int m_tiles = Mf / BM, n_tiles = Nf / BN;
  const int per_e = m_tiles * n_tiles;
  const int total = experts * per_e;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const int e = tile / per_e;
    const int rem = tile % per_e;
    const int mt = rem / n_tiles, nt = rem % n_tiles;
    const int kb0 = prefix[e], nk = prefix[e + 1] - prefix[e];

    const int lr = tid >> 3, lc = (tid & 7) * 16;
    const uint8_t* gp[4];
    const uint8_t* gq[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      gp[s] = p + (size_t)(mt * BM + lr + 32 * s) * padded + lc;
      gq[s] = q + (size_t)(nt * BN + lr + 32 * s) * padded + lc;
    }
    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    uint4 ra[4], rb[4];
    float rs = 0.0f;
    auto fetch = [&](int kb) {
      const size_t koff = (size_t)(kb0 + kb) * 128;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        ra[s] = *(const uint4*)(gp[s] + koff);
        rb[s] = *(const uint4*)(gq[s] + koff);
      }
      if (tid < BM) rs = p_scale[(size_t)(kb0 + kb) * Mf + mt * BM + tid];
      else rs = q_scale[(size_t)(kb0 + kb) * Nf + nt * BN + tid - BM];
    };
    auto stash = [&](int buf) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        *(uint4*)&lds.a[buf][(lr + 32 * s) * PITCH + lc] = ra[s];
        *(uint4*)&lds.b[buf][(lr + 32 * s) * PITCH + lc] = rb[s];
      }
      if (tid < BM) lds.sa[buf][tid] = rs; else lds.sb[buf][tid - BM] = rs;
    };
    if (nk > 0) {
      fetch(0);
      stash(0);
    }
    __syncthreads();
    for (int kb = 0; kb < nk; ++kb) {
      const int buf = kb & 1;
      if (kb + 1 < nk) fetch(kb + 1);
      {
        v8i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = lds_frag(lds.a[buf], wm * 64 + i * 16 + (lane & 15), lane);
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = lds_frag(lds.b[buf], wn * 64 + j * 16 + (lane & 15), lane);
        float rsc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float4 s4 = *(const float4*)&lds.sa[buf][wm * 64 + i * 16 + 4 * (lane >> 4)];
          rsc[i][0] = s4.x; rsc[i][1] = s4.y; rsc[i][2] = s4.z; rsc[i][3] = s4.w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float cs = lds.sb[buf][wn * 64 + j * 16 + (lane & 15)];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v4f pr = mfma_f8(af[i], bf[j]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(pr[r], rsc[i][r] * cs, acc[i][j][r]);
          }
        }
      }
      if (kb + 1 < nk) stash(buf ^ 1);
      __syncthreads();
    }

    float* stage = (float*)&lds;
    constexpr int SP = BN + 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          stage[(wm * 64 + i * 16 + 4 * (lane >> 4) + r) * SP + wn * 64 + j * 16 + (lane & 15)] =
              acc[i][j][r];
    __syncthreads();
    const size_t base = ((size_t)e * Mf + mt * BM) * Nf + nt * BN;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int idx = s * kThreads + tid;
      const int r = idx >> 4, c8 = (idx & 15) * 8;
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = stage[r * SP + c8 + i];
      const size_t off = base + (size_t)r * Nf + c8;
      if (out_fp32) {
        float* o = (float*)out + off;
        *(float4*)o = make_float4(v[0], v[1], v[2], v[3]);
        *(float4*)(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
      } else {
        uint4 o;
        o.x = pack_bf16x2(v[0], v[1]);
        o.y = pack_bf16x2(v[2], v[3]);
        o.z = pack_bf16x2(v[4], v[5]);
        o.w = pack_bf16x2(v[6], v[7]);
        *(uint4*)((uint16_t*)out + off) = o;
      }
    }
    __syncthreads();
  }
}

int persistent_grid(int tiles) {
  static int cus[64] = {0};
  int dev = 0;
  hipGetDevice(&dev);
  if (dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  int g = cus[dev] * 2;
  return tiles < g ? tiles : g;
}

}  // namespace

int mi355x_gemm_v2_launch(const uint8_t* a, const float* a_scale, int rows, const uint8_t* w,
                          const float* w_scale, int w_scale_t, int experts, int n, int k,
                          const int32_t* offsets, int interleave, const void* addend, void* out,
                          uint8_t* act_q, float* act_scales, float limit, const void* lora_z,
                          const void* lora_b, int lora_rank, void* stream,
                          const int32_t* a_rows = nullptr, int a_total = 0, int a_rows_div = 1);
int mi355x_gemm_v2_kmajor_launch(const uint8_t* a, const float* a_scale, int rows,
                                 const uint8_t* w, const float* w_scale, int experts, int n, int k,
                                 const int32_t* offsets, void* out, void* stream,
                                 const int32_t* a_rows = nullptr, int a_total = 0, int a_rows_div = 1);

int mi355x_gemm_v2_rowwise_launch(const uint8_t* a, const float* a_scale, int rows,
                                  const uint8_t* w, const float* w_scale, int experts, int n,
                                  int k, const int32_t* offsets, const void* lora_z,
                                  const void* lora_b, int lora_rank, void* out, void* stream,
                                  const int32_t* a_rows = nullptr, int a_total = 0, int a_rows_div = 1);

int mi355x_wgrad_v2_launch(const uint8_t* p, const float* p_scale, int m_features,
                           const uint8_t* q, const float* q_scale, int n_features, int padded,
                           const int32_t* offsets, int experts, void* out, int out_fp32,
                           void* stream);

extern "C" int mi355x_gemm_fp8_block(const uint8_t* a, const float* a_scale, int rows,
                                     const uint8_t* w, const float* w_scale, int w_scale_t,
                                     int experts, int n, int k, const int32_t* offsets,
                                     int interleave, const void* addend, void* out,
                                     void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "gemm: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % BN == 0, "gemm: N must be a multiple of %d, got %d", BN, n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE(!interleave || (n / 2) % 64 == 0,
                 "gemm: a gate/up weight needs halves that are multiples of 64");
  MI355X_REQUIRE(rows >= 0, "gemm: negative rows");
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_launch(a, a_scale, rows, w, w_scale, w_scale_t, experts, n, k,
                                       offsets, interleave, addend, out, nullptr, nullptr, 0.0f,
                                       nullptr, nullptr, 0, stream);
  if (v2 <= 0) return v2;
  const int upper = ((rows + BM - 1) / BM + experts) * (n / BN);
  hipLaunchKernelGGL(grouped_gemm_kernel, dim3(persistent_grid(upper)), dim3(kThreads), 0,
                     (hipStream_t)stream, a, a_scale, rows, w, w_scale, w_scale_t, experts, n, k,
                     offsets, interleave, (const uint16_t*)addend, (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_block_kmajor(const uint8_t* a, const float* a_scale, int rows,
                                            const uint8_t* w, const float* w_scale, int experts,
                                            int n, int k, const int32_t* offsets, void* out,
                                            void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts,
                 "gemm_kmajor: experts must be in [1, %d]", kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0, "gemm_kmajor: N must be a multiple of 256, got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_kmajor: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE(rows >= 0, "gemm_kmajor: negative rows");
  MI355X_REQUIRE((uint64_t)(k - 1) * (uint64_t)n + 256 < (1ull << 32),
                 "gemm_kmajor: a weight slice beyond 32-bit offsets");
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_kmajor_launch(a, a_scale, rows, w, w_scale, experts, n, k, offsets,
                                              out, stream);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm_kmajor: shape outside the pipelined kernel");
  return MI355X_OK;
}

// Gathered-A forms: GEMM row r (expert-sorted, offsets) reads row
// a_rows[r] of a [a_total, K] and its 1x128 scales a_scale[a_total][K/128]
// (token-major, as mi355x_quantize_token_rows_fp8 writes them)
// (the activation quantized once per token; a_rows = the token of each
// routed row). Pipelined kernel only (N a multiple of 256).
static int gathered_checks(int a_total, const int32_t* a_rows, int a_rows_div, int rows, int k) {
  MI355X_REQUIRE(a_rows != nullptr && a_total > 0, "gemm gathered: a_rows and a_total required");
  MI355X_REQUIRE(a_rows_div >= 1 && (uint64_t)a_total * (uint64_t)a_rows_div < (1ull << 31),
                 "gemm gathered: a_rows_div must be >= 1 with a_total * a_rows_div < 2^31");
  MI355X_REQUIRE((uint64_t)a_total * (uint64_t)k < (1ull << 32),
                 "gemm gathered: gathered rows beyond 32-bit offsets");
  MI355X_REQUIRE(rows >= 0, "gemm gathered: negative rows");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_block_gathered(const uint8_t* a, const float* a_scale, int a_total,
                                              const int32_t* a_rows, int a_rows_div, int rows, const uint8_t* w,
                                              const float* w_scale, int experts, int n, int k,
                                              const int32_t* offsets, int interleave, void* out,
                                              void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "gemm: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0, "gemm gathered: N must be a multiple of 256, got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE(!interleave || (n / 2) % 128 == 0,
                 "gemm gathered: a gate/up weight needs halves that are multiples of 128");
  const int c = gathered_checks(a_total, a_rows, a_rows_div, rows, k);
  if (c != MI355X_OK) return c;
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_launch(a, a_scale, rows, w, w_scale, 0, experts, n, k, offsets,
                                       interleave, nullptr, out, nullptr, nullptr, 0.0f, nullptr,
                                       nullptr, 0, stream, a_rows, a_total, a_rows_div);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm gathered: shape outside the pipelined kernel");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_block_kmajor_gathered(const uint8_t* a, const float* a_scale,
                                                     int a_total, const int32_t* a_rows, int a_rows_div, int rows,
                                                     const uint8_t* w, const float* w_scale,
                                                     int experts, int n, int k,
                                                     const int32_t* offsets, void* out,
                                                     void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts,
                 "gemm_kmajor: experts must be in [1, %d]", kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0, "gemm_kmajor: N must be a multiple of 256, got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_kmajor: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE((uint64_t)(k - 1) * (uint64_t)n + 256 < (1ull << 32),
                 "gemm_kmajor: a weight slice beyond 32-bit offsets");
  const int c = gathered_checks(a_total, a_rows, a_rows_div, rows, k);
  if (c != MI355X_OK) return c;
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_kmajor_launch(a, a_scale, rows, w, w_scale, experts, n, k, offsets,
                                              out, stream, a_rows, a_total, a_rows_div);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm_kmajor: shape outside the pipelined kernel");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_rowwise_gathered(const uint8_t* a, const float* a_scale,
                                                int a_total, const int32_t* a_rows, int a_rows_div, int rows,
                                                const uint8_t* w, const float* w_scale,
                                                int experts, int n, int k,
                                                const int32_t* offsets, void* out, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "gemm_rowwise: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0, "gemm_rowwise: N must be a multiple of 256, got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_rowwise: K must be a multiple of %d, got %d", BK, k);
  const int c = gathered_checks(a_total, a_rows, a_rows_div, rows, k);
  if (c != MI355X_OK) return c;
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_rowwise_launch(a, a_scale, rows, w, w_scale, experts, n, k, offsets,
                                               nullptr, nullptr, 0, out, stream, a_rows, a_total, a_rows_div);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm_rowwise gathered: shape outside the pipelined kernel");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_rowwise(const uint8_t* a, const float* a_scale, int rows,
                                       const uint8_t* w, const float* w_scale, int experts, int n,
                                       int k, const int32_t* offsets, void* out, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "gemm_rowwise: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0, "gemm_rowwise: N must be a multiple of 256, got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_rowwise: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE(rows >= 0, "gemm_rowwise: negative rows");
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_rowwise_launch(a, a_scale, rows, w, w_scale, experts, n, k,
                                               offsets, nullptr, nullptr, 0, out, stream);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm_rowwise: shape outside the pipelined kernel");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_rowwise_lora(const uint8_t* a, const float* a_scale, int rows,
                                            const uint8_t* w, const float* w_scale, int experts,
                                            int n, int k, const int32_t* offsets,
                                            const void* lora_z, const void* lora_b, int lora_rank,
                                            void* out, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts,
                 "gemm_rowwise_lora: experts must be in [1, %d]", kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0, "gemm_rowwise_lora: N must be a multiple of 256, got %d",
                 n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_rowwise_lora: K must be a multiple of %d", BK);
  MI355X_REQUIRE(lora_rank >= 16 && lora_rank <= 256 && lora_rank % 16 == 0,
                 "gemm_rowwise_lora: rank must be a multiple of 16 in [16, 256], got %d",
                 lora_rank);
  MI355X_REQUIRE(lora_z != nullptr && lora_b != nullptr, "gemm_rowwise_lora: z and b are required");
  MI355X_REQUIRE(rows >= 0, "gemm_rowwise_lora: negative rows");
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_rowwise_launch(a, a_scale, rows, w, w_scale, experts, n, k,
                                               offsets, lora_z, lora_b, lora_rank, out, stream);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm_rowwise_lora: shape outside the pipelined kernel");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_block_lora(const uint8_t* a, const float* a_scale, int rows,
                                          const uint8_t* w, const float* w_scale, int w_scale_t,
                                          int experts, int n, int k, const int32_t* offsets,
                                          int interleave, const void* lora_z, const void* lora_b,
                                          int lora_rank, void* out, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "gemm_lora: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % 256 == 0 && (!interleave || (n / 2) % 128 == 0),
                 "gemm_lora: N must be a multiple of 256 (2I of 128), got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_lora: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE(lora_rank > 0 && lora_rank % 16 == 0 && lora_rank <= 256,
                 "gemm_lora: the (padded) rank must be a multiple of 16 in [16, 256], got %d",
                 lora_rank);
  MI355X_REQUIRE(lora_z != nullptr && lora_b != nullptr, "gemm_lora: z and b are required");
  MI355X_REQUIRE(rows >= 0, "gemm_lora: negative rows");
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_launch(a, a_scale, rows, w, w_scale, w_scale_t, experts, n, k,
                                       offsets, interleave, nullptr, out, nullptr, nullptr, 0.0f,
                                       lora_z, lora_b, lora_rank, stream);
  if (v2 < 0) return v2;
  MI355X_REQUIRE(v2 == 0, "gemm_lora: shape outside the pipelined kernel");
  return MI355X_OK;
}

extern "C" int mi355x_gemm_fp8_block_swiglu(const uint8_t* a, const float* a_scale, int rows,
                                            const uint8_t* w, const float* w_scale, int experts,
                                            int n, int k, const int32_t* offsets,
                                            const void* addend, float limit, void* h,
                                            uint8_t* act_q, float* act_scales, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "gemm_swiglu: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(n > 0 && n % BN == 0 && (n / 2) % 128 == 0,
                 "gemm_swiglu: 2I must be a multiple of 256, got %d", n);
  MI355X_REQUIRE(k > 0 && k % BK == 0, "gemm_swiglu: K must be a multiple of %d, got %d", BK, k);
  MI355X_REQUIRE(rows >= 0, "gemm_swiglu: negative rows");
  if (rows == 0) return MI355X_OK;
  const int v2 = mi355x_gemm_v2_launch(a, a_scale, rows, w, w_scale, 0, experts, n, k, offsets, 1,
                                       addend, h, act_q, act_scales, limit, nullptr, nullptr, 0,
                                       stream);
  if (v2 <= 0) return v2;
  // Shapes outside the pipelined kernel: the GEMM, then the SwiGLU pass.
  const int rc = mi355x_gemm_fp8_block(a, a_scale, rows, w, w_scale, 0, experts, n, k, offsets, 1,
                                       addend, h, stream);
  if (rc != MI355X_OK) return rc;
  return mi355x_swiglu_quantize_fp8(h, rows, n / 2, limit, act_q, act_scales, nullptr, stream);
}

extern "C" int mi355x_gemm_fp8_block_wgrad(const uint8_t* p, const float* p_scale,
                                           int m_features, const uint8_t* q,
                                           const float* q_scale, int n_features, int padded,
                                           const int32_t* offsets, int experts, void* out,
                                           int out_fp32, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= kMaxExperts, "wgrad: experts must be in [1, %d]",
                 kMaxExperts);
  MI355X_REQUIRE(m_features > 0 && m_features % BM == 0 && n_features > 0 && n_features % BN == 0,
                 "wgrad: feature counts must be multiples of 128");
  MI355X_REQUIRE(padded % 128 == 0, "wgrad: padded rows must be a multiple of 128");
  const int v2 = mi355x_wgrad_v2_launch(p, p_scale, m_features, q, q_scale, n_features, padded,
                                        offsets, experts, out, out_fp32, stream);
  if (v2 <= 0) return v2;
  const int tiles = experts * (m_features / BM) * (n_features / BN);
  hipLaunchKernelGGL(wgrad_gemm_kernel, dim3(persistent_grid(tiles)), dim3(kThreads), 0,
                     (hipStream_t)stream, p, p_scale, m_features, q, q_scale, n_features, padded,
                     offsets, experts, out, out_fp32);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
