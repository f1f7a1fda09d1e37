// Grouped block-FP8 GEMM, pipelined form (N a multiple of 256): projection
// (y = x @ W^T), input gradient (dx = dy @ W through the transposed copy) and
// the gate/up-interleaved up projection. See gemm_pipe.h for the tiling.
#include <type_traits>

#include "gemm_pipe.h"

using namespace pipe;

namespace {

constexpr int kMaxExperts = 512;
constexpr int STAGE_PITCH = BN + 4;  // fp32 epilogue staging row pitch
static_assert(48 * STAGE_PITCH * 4 <= STAGE_BYTES, "epilogue rows per stage");

__global__ void __launch_bounds__(kThreads, 1) grouped_gemm_v2_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ a_scale, int rows,
    const uint8_t* __restrict__ w, const float* __restrict__ w_scale, int w_scale_t, int experts,
    int N, int K, const int32_t* __restrict__ offsets, int interleave,
    const uint16_t* __restrict__ addend, uint16_t* __restrict__ out) {
  // Three distinct LDS objects, one per stage, selected with compile-time
  // indices only: the compiler then proves an in-flight direct load into one
  // stage never aliases the LDS reads of another, and adds no blanket
  // vmcnt(0) before them.
  __shared__ __align__(1024) uint8_t st0[STAGE_BYTES];
  __shared__ __align__(1024) uint8_t st1[STAGE_BYTES];
  __shared__ __align__(1024) uint8_t st2[STAGE_BYTES];
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ int tmp[kThreads];
  tile_prefix(offsets, experts, BM, prefix, tmp);
  const int total = prefix[experts] * (N / BN);
  const int n_tiles = N / BN;
  const int nk = K / BK;
  const int kbw = K / 128, nbw = N / 128, half_n = N / 2;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  for (int round = 0;; ++round) {
    const int tile = tile_of(round, blockIdx.x, gridDim.x);
    if (tile >= total) break;
    const int mt = tile / n_tiles, nt = tile % n_tiles;
    const int e = find_expert(prefix, experts, mt);
    const int row0 = offsets[e] + (mt - prefix[e]) * BM;
    const int nvalid = min(BM, offsets[e + 1] - row0);
    const int j0 = nt * 128;  // interleave: gate/up pair index of the tile
    const uint8_t* wexp = w + (size_t)e * N * K;

    // Per-lane direct-load sources (byte offsets) for this tile.
    uint32_t offa[A_LOADS], offb[B_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int r = (wave * A_LOADS + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ swz(r);
      offa[i] = (uint32_t)min(row0 + r, rows - 1) * (uint32_t)K + 16 * c;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int tr = (wave * B_LOADS + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ swz(tr);
      int wr;
      if (interleave) {
        const int q = tr >> 6, jj = j0 + 64 * (q >> 1) + (tr & 63);
        wr = (q & 1) ? half_n + jj : jj;
      } else {
        wr = nt * BN + tr;
      }
      offb[i] = (uint32_t)wr * (uint32_t)K + 16 * c;
    }
    const int sa_row = min(row0 + wave * 32 + (lane & 31), rows - 1);
    // Weight-block scale columns of this wave's two 64-column halves.
    const int nb_lo = interleave ? j0 / 128 : 2 * nt + wn;
    const int nb_hi = interleave ? (half_n + j0) / 128 : 2 * nt + wn;

    auto issue = [&](auto stage_c, int kb) {
      constexpr int stage = decltype(stage_c)::value;
      uint8_t* base = stage == 0 ? st0 : (stage == 1 ? st1 : st2);
      const size_t koff = (size_t)kb * BK;
      const uint8_t* abase = a + koff;
      const uint8_t* bbase = wexp + koff;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) dma16(abase, offa[i], base + (wave * A_LOADS + i) * 1024);
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) dma16(bbase, offb[i], base + A_BYTES + (wave * B_LOADS + i) * 1024);
      if (lane < 32)
        dma4(a_scale + (size_t)kb * rows, 4u * (uint32_t)sa_row, base + A_BYTES + B_BYTES + wave * 128);
    };
    auto wscale = [&](int nb, int kb) {
      return w_scale_t ? w_scale[((size_t)e * kbw + kb) * nbw + nb]
                       : w_scale[((size_t)e * nbw + nb) * kbw + kb];
    };

    v4f acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    auto step = [&](auto stage_c, int kb) {
      constexpr int S = decltype(stage_c)::value;
      if (kb + 1 < nk) wait_and_sync<A_LOADS + B_LOADS + 1>();
      else wait_and_sync<0>();
      if (kb + 2 < nk) issue(std::integral_constant<int, (S + 2) % kStages>{}, kb + 2);
      const uint8_t* base = S == 0 ? st0 : (S == 1 ? st1 : st2);
      const uint8_t* ta = base;
      const uint8_t* tb = base + A_BYTES;
      const float* sa = (const float*)(base + A_BYTES + B_BYTES);
      const float sb_lo = wscale(nb_lo, kb), sb_hi = wscale(nb_hi, kb);
      v8i af[4];
      float s4[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        af[i] = frag(ta, wm * 64 + i * 16 + (lane & 15), lane);
        float4 v = *(const float4*)&sa[wm * 64 + i * 16 + 4 * (lane >> 4)];
        s4[i][0] = v.x; s4[i][1] = v.y; s4[i][2] = v.z; s4[i][3] = v.w;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float sb = h ? sb_hi : sb_lo;
        v8i bf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = frag(tb, wn * 128 + (h * 4 + j) * 16 + (lane & 15), lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float sc[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] = s4[i][r] * sb;
          v4f p[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) p[j] = mfma(af[i], bf[j]);
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][h * 4 + j][r] = fmaf(p[j][r], sc[r], acc[i][h * 4 + j][r]);
        }
      }
    };

    issue(std::integral_constant<int, 0>{}, 0);
    if (nk > 1) issue(std::integral_constant<int, 1>{}, 1);
    for (int kb = 0; kb < nk; kb += kStages) {
      step(std::integral_constant<int, 0>{}, kb);
      if (kb + 1 < nk) step(std::integral_constant<int, 1>{}, kb + 1);
      if (kb + 2 < nk) step(std::integral_constant<int, 2>{}, kb + 2);
    }

    // Epilogue: fp32 tile staged in LDS (interleave mapping applied), then
    // 16-byte row stores (+ addend), rounded once to bf16.
    sync_all();
    // rows 0-47 in stage 0, 48-95 in stage 1, 96-127 in stage 2
    auto stage_row = [&](int row) -> float* {
      uint8_t* base = row < 48 ? st0 : (row < 96 ? st1 : st2);
      return (float*)base + (row % 48) * STAGE_PITCH;
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int jb = 0; jb < 8; ++jb) {
        const int tc = wn * 128 + jb * 16 + (lane & 15);
        int oc = tc;
        if (interleave) {
          const int q = tc >> 6, jl = 64 * (q >> 1) + (tc & 63);
          oc = 2 * jl + (q & 1);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * 64 + i * 16 + 4 * (lane >> 4) + r;
          stage_row(row)[oc] = acc[i][jb][r];
        }
      }
    }
    sync_all();
    const int col0 = nt * BN;
#pragma unroll 4
    for (int idx = tid; idx < BM * (BN / 8); idx += kThreads) {
      const int r = idx / (BN / 8), c8 = (idx % (BN / 8)) * 8;
      if (r < nvalid) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = stage_row(r)[c8 + i];
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
    sync_all();
  }
}

int cu_count() {
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
  return cus[dev];
}

}  // namespace

// Launches the pipelined kernel; returns 1 if the shape is not its form
// (N % 256 != 0), in which case the caller uses the general kernel.
int mi355x_gemm_v2_launch(const uint8_t* a, const float* a_scale, int rows, const uint8_t* w,
                          const float* w_scale, int w_scale_t, int experts, int n, int k,
                          const int32_t* offsets, int interleave, const void* addend, void* out,
                          void* stream) {
  if (n % BN != 0 || experts > kMaxExperts || (interleave && (n / 2) % 128 != 0)) return 1;
  const int upper = ((rows + BM - 1) / BM + experts) * (n / BN);
  const int grid = upper < cu_count() ? upper : cu_count();
  hipLaunchKernelGGL(grouped_gemm_v2_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a,
                     a_scale, rows, w, w_scale, w_scale_t, experts, n, k, offsets, interleave,
                     (const uint16_t*)addend, (uint16_t*)out);
  MI355X_LAUNCH_CHECK();
  return 0;
}
