// Grouped weight-gradient GEMM, pipelined form (both feature counts
// multiples of 256):
//   out[e][m][n] = sum over expert e's padded rows k of P[m][k] * Q[n][k]
// with P, Q the feature-major e4m3 operands written by the transposing
// quantizer and one power-of-two descale per (feature, 128-row block).
//
// Same main loop as the grouped GEMM (gemm_pipe.h: 256 x 256 tile, 8 waves,
// direct-to-LDS loads, two stages) with one difference: both operands carry
// per-row scales that are powers of two, so the MFMA applies them itself
// (v_mfma_scale_f32_16x16x128_f8f6f4 with E8M0 scales = the fp32 exponent
// byte) and accumulates across K blocks in place: no VALU work in the loop.
// Hardware operand layout (measured on MI355X): lane l of a 16x16x128
// fragment holds K bytes [16g, 16g+16) and [64+16g, 64+16g+16), g = l / 16,
// and the scale of (row m, 32-wide K block b) is taken from lane 16b + m; a
// scale constant over the 128 K values means each lane passes its own row's.
#include "gemm_pipe.h"

using namespace pipe;

namespace {

constexpr int kMaxExperts = 512;

// q feature behind B-tile row tr: MFMA column c of block jb feeds output
// column c * 8 + jb of the wave's 128, so a lane's eight accumulator blocks
// are eight consecutive output columns.
__device__ __forceinline__ int feature_col(int tr, int nt) {
  const int part = tr >> 7, local = tr & 127;
  return nt * BN + part * 128 + (local & 15) * 8 + (local >> 4);
}

__device__ __forceinline__ int e8m0(float pow2_scale) { return __float_as_int(pow2_scale) >> 23; }

__device__ __forceinline__ v4f mfma_e8(v8i a, v8i b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

struct WTile {
  int e, mt, nt, k0, nk;  // expert, tile coordinates, first padded block, blocks
  int rot;                // K-step rotation (see wdescribe)
};

__device__ __forceinline__ WTile wdescribe(const int* prefix, int per_e, int n_tiles, int tile) {
  WTile t;
  t.e = __builtin_amdgcn_readfirstlane(tile / per_e);
  const int rem = tile - t.e * per_e;
  t.mt = __builtin_amdgcn_readfirstlane(rem / n_tiles);
  t.nt = __builtin_amdgcn_readfirstlane(rem - t.mt * n_tiles);
  t.k0 = __builtin_amdgcn_readfirstlane(prefix[t.e]);
  t.nk = __builtin_amdgcn_readfirstlane(prefix[t.e + 1] - prefix[t.e]);
  // Tiles sharing an operand panel run together on neighbouring CUs; each
  // starts at a different K step so that one takes a step's L2 miss and the
  // others hit later instead of all waiting on the same miss.
  t.rot = t.nk > 0 ? __builtin_amdgcn_readfirstlane((tile * 7) % t.nk) : 0;
  return t;
}

__global__ void __launch_bounds__(kThreads, 2) wgrad_v2_kernel(
    const uint8_t* __restrict__ p, const float* __restrict__ p_scale, int Mf,
    const uint8_t* __restrict__ q, const float* __restrict__ q_scale, int Nf, int padded,
    const int32_t* __restrict__ offsets, int experts, void* __restrict__ out, int out_fp32) {
  __shared__ __align__(1024) uint8_t smem[kStages * STAGE_BYTES];
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ int tmp[kThreads];
  tile_prefix(offsets, experts, 128, prefix, tmp);  // padded 128-row blocks per expert
  const int n_tiles = Nf / BN;
  const int per_e = (Mf / BM) * n_tiles;
  const int total = experts * per_e;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 wave grid

  auto issue = [&](const WTile& t, int step, int stage) {
    const int kb = __builtin_amdgcn_readfirstlane(step + t.rot < t.nk ? step + t.rot : step + t.rot - t.nk);
    uint8_t* base = smem + stage * STAGE_BYTES;
    const size_t kblock = (size_t)(t.k0 + kb);
    const uint8_t* abase = p + kblock * 128;
    const uint8_t* bbase = q + kblock * 128;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int r = (wave * A_LOADS + i) * 8 + (lane >> 3);
      const uint32_t off = (uint32_t)(t.mt * BM + r) * (uint32_t)padded + 16 * ((lane & 7) ^ swz(r));
      dma16(abase, off, base + (wave * A_LOADS + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int tr = (wave * B_LOADS + i) * 8 + (lane >> 3);
      const uint32_t off = (uint32_t)feature_col(tr, t.nt) * (uint32_t)padded + 16 * ((lane & 7) ^ swz(tr));
      dma16(bbase, off, base + A_BYTES + (wave * B_LOADS + i) * 1024);
    }
    // Scales of this K block, stored in lane order: LDS slot wm*64 + c*4 + i
    // holds P row wm*64 + i*16 + c, slot wn*128 + c*8 + jb holds the Q row
    // of B-tile row wn*128 + jb*16 + c, so that a fragment lane (c = lane %
    // 16) fetches its 4 row scales and 8 column scales with 16-byte reads.
    // Waves 0-3 load the P scales, waves 4-7 the Q scales.
    uint8_t* sbase = base + A_BYTES + B_BYTES;
    if (wave < 4) {
      const int slot = wave * 64 + lane;
      const int row = (slot & ~63) + (slot & 3) * 16 + ((slot >> 2) & 15);
      dma4(p_scale + kblock * Mf + t.mt * BM, 4u * (uint32_t)row, sbase + wave * 256);
    } else {
      const int slot = (wave - 4) * 64 + lane;
      const int tr = (slot & ~127) + (slot & 7) * 16 + ((slot >> 3) & 15);
      dma4(q_scale + kblock * Nf, 4u * (uint32_t)feature_col(tr, t.nt),
           sbase + SA_BYTES + (wave - 4) * 256);
    }
  };

  // XCD-affine order: workgroup b runs on XCD b % 8, and XCD x takes a
  // contiguous range of the expert-major tile list holding 1/8 of the total
  // work (a tile costs its expert's K blocks), so an expert's operand panels
  // are fetched into one or two XCD L2s instead of all eight. The 8 x G/8
  // workgroups of an XCD take its range round-robin. Needs a grid that is a
  // multiple of 8; otherwise plain order.
  const bool affine = (gridDim.x & 7) == 0;
  const int xcd = blockIdx.x & 7, cu = blockIdx.x >> 3, per_xcd = gridDim.x >> 3;
  auto range_start = [&](int x) -> int {  // first tile of XCD x's range
    if (x <= 0) return 0;
    if (x >= 8) return total;
    const long long bound = (long long)per_e * prefix[experts] * x / 8;
    int lo = 0, hi = experts - 1;  // last e with cost before it <= bound
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((long long)per_e * prefix[mid] <= bound) lo = mid; else hi = mid - 1;
    }
    const int nk = prefix[lo + 1] - prefix[lo];
    const long long rem = bound - (long long)per_e * prefix[lo];
    const long long j = nk > 0 ? (rem + nk - 1) / nk : per_e;
    return lo * per_e + (int)(j < per_e ? j : per_e);
  };
  const int first = __builtin_amdgcn_readfirstlane(affine ? range_start(xcd) : 0);
  const int last = __builtin_amdgcn_readfirstlane(affine ? range_start(xcd + 1) : total);
  auto tile_at = [&](int r) -> int {
    if (!affine) return tile_of(r, blockIdx.x, gridDim.x);
    const int t = first + r * per_xcd + cu;
    return t < last ? t : total;
  };
  int round = 0;
  int tile = tile_at(0);
  if (tile >= total) return;
  WTile ct = wdescribe(prefix, per_e, n_tiles, tile);
  bool issued = false;  // whether the current tile's first step is in flight
  int stage = 0;
  for (;;) {
    if (!issued && ct.nk > 0) issue(ct, 0, stage);
    issued = false;
    const int next_tile = tile_at(round + 1);
    v4f acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    for (int kb = 0; kb < ct.nk; ++kb) {
      wait_and_sync<0>();
      if (kb + 1 < ct.nk) {
        issue(ct, kb + 1, stage ^ 1);
      } else if (next_tile < total) {
        const WTile nt = wdescribe(prefix, per_e, n_tiles, next_tile);
        if (nt.nk > 0) {
          issue(nt, 0, stage ^ 1);
          issued = true;
        }
      }
      const uint8_t* base = smem + stage * STAGE_BYTES;
      const uint8_t* ta = base;
      const uint8_t* tb = base + A_BYTES;
      const float* sa = (const float*)(base + A_BYTES + B_BYTES);
      const float* sb = sa + BM;
      const int c = lane & 15;
      const float4 sa4 = *(const float4*)&sa[wm * 64 + c * 4];
      const float4 sb_lo = *(const float4*)&sb[wn * 128 + c * 8];
      const float4 sb_hi = *(const float4*)&sb[wn * 128 + c * 8 + 4];
      // Reads in the order the first MFMAs consume them (the step starts
      // with every wave of the CU reading at once, so what comes first
      // decides when the matrix cores start), B fragments through a
      // three-slot ring, read two blocks ahead.
      v8i af[4], bf[3];
      bf[0] = frag(tb, wn * 128 + c, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = frag(ta, wm * 64 + i * 16 + c, lane);
      bf[1] = frag(tb, wn * 128 + 16 + c, lane);
      __builtin_amdgcn_sched_barrier(0);
      // Exponent bytes after the fragment reads are in flight: waiting for
      // the scales then does not hold back the fragment reads.
      const int ea[4] = {e8m0(sa4.x), e8m0(sa4.y), e8m0(sa4.z), e8m0(sa4.w)};
      const int eb[8] = {e8m0(sb_lo.x), e8m0(sb_lo.y), e8m0(sb_lo.z), e8m0(sb_lo.w),
                         e8m0(sb_hi.x), e8m0(sb_hi.y), e8m0(sb_hi.z), e8m0(sb_hi.w)};
#pragma unroll
      for (int jb = 0; jb < 8; ++jb) {
        if (jb + 2 < 8) bf[(jb + 2) % 3] = frag(tb, wn * 128 + (jb + 2) * 16 + c, lane);
        // Keep the read ahead of this block's MFMAs (the scheduler would
        // otherwise sink it to shorten live ranges, leaving one group of
        // MFMAs to cover the LDS latency).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][jb] = mfma_e8(af[i], bf[jb % 3], acc[i][jb], ea[i], eb[jb]);
        __builtin_amdgcn_sched_barrier(0);
      }
      stage ^= 1;
    }

    // Epilogue from registers: lane (row, 8 consecutive columns).
    const size_t row0 = (size_t)ct.e * Mf + ct.mt * BM + wm * 64;
    const size_t col0 = (size_t)ct.nt * BN + wn * 128 + (lane & 15) * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int lrow = i * 16 + 4 * (lane >> 4) + r;
        const size_t off = (row0 + lrow) * Nf + col0;
        if (out_fp32) {
          float* o = (float*)out + off;
          store_stream(o, make_uint4(__float_as_uint(acc[i][0][r]), __float_as_uint(acc[i][1][r]), __float_as_uint(acc[i][2][r]), __float_as_uint(acc[i][3][r])));
          store_stream(o + 4, make_uint4(__float_as_uint(acc[i][4][r]), __float_as_uint(acc[i][5][r]), __float_as_uint(acc[i][6][r]), __float_as_uint(acc[i][7][r])));
        } else {
          uint4 o;
          o.x = pack_bf16x2(acc[i][0][r], acc[i][1][r]);
          o.y = pack_bf16x2(acc[i][2][r], acc[i][3][r]);
          o.z = pack_bf16x2(acc[i][4][r], acc[i][5][r]);
          o.w = pack_bf16x2(acc[i][6][r], acc[i][7][r]);
          store_stream((uint16_t*)out + off, o);
        }
      }
    }
    if (next_tile >= total) break;
    ++round;
    ct = wdescribe(prefix, per_e, n_tiles, next_tile);
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
// (feature counts not multiples of 256, or operands beyond 32-bit offsets),
// in which case the caller uses the general kernel.
int mi355x_wgrad_v2_launch(const uint8_t* p, const float* p_scale, int m_features,
                           const uint8_t* q, const float* q_scale, int n_features, int padded,
                           const int32_t* offsets, int experts, void* out, int out_fp32,
                           void* stream) {
  if (m_features % BM != 0 || n_features % BN != 0 || experts > kMaxExperts) return 1;
  if ((uint64_t)m_features * (uint64_t)padded >= (1ull << 32) ||
      (uint64_t)n_features * (uint64_t)padded >= (1ull << 32))
    return 1;
  const int total = experts * (m_features / BM) * (n_features / BN);
  const int grid = total < cu_count() ? total : cu_count();
  hipLaunchKernelGGL(wgrad_v2_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, p,
                     p_scale, m_features, q, q_scale, n_features, padded, offsets, experts, out,
                     out_fp32);
  MI355X_LAUNCH_CHECK();
  return 0;
}
