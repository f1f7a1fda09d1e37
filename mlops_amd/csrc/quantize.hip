// FP8 (OCP e4m3) quantizers of the block-FP8 MoE path and the routed SwiGLU
// backward row pass. All of them are HBM-bound byte/element work: each reads
// its source once with 16-byte vector loads and writes e4m3 with 8- or
// 16-byte stores; 128-element scale groups are formed by 16-lane shuffles.
#include "common.h"

namespace {

// ---------------------------------------------------------------------------
// 128x128 weight blocks. One block per (expert, block row, block column); a
// 16-lane group reads one 256-byte row slice, 16 rows per pass, 8 passes.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* v) { unpack_bf16x8(load_stream(p), v); }
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* v) {
  float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <typename T>
__global__ void __launch_bounds__(256) weight_blocks_kernel(
    const T* __restrict__ w, int out, int in, int bo_count, int bi_count,
    uint8_t* __restrict__ q, float* __restrict__ scale, uint8_t* __restrict__ q_t) {
  __shared__ float red[4];
  __shared__ uint8_t tile[128][128 + 8];
  const int e = blockIdx.z, bo = blockIdx.y, bi = blockIdx.x;
  const int lane16 = threadIdx.x & 15, rsub = threadIdx.x >> 4;
  const int col = bi * 128 + lane16 * 8;
  const size_t ebase = (size_t)e * out * in;
  float v[8][8];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int row = bo * 128 + p * 16 + rsub;
    if (row < out && col < in) {
      load8<T>(w + ebase + (size_t)row * in + col, v[p]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[p][i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[p][i]));
  }
  amax = group_amax<64>(amax);
  if (lane_id() == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(amax / kE4M3Max, kMinScale);
  if (threadIdx.x == 0) scale[((size_t)e * bo_count + bo) * bi_count + bi] = s;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int row = bo * 128 + p * 16 + rsub;
    uint2 packed = quant8(v[p], s);
    if (row < out && col < in) store_stream8(q + ebase + (size_t)row * in + col, packed);
    if (q_t != nullptr) *(uint2*)&tile[p * 16 + rsub][lane16 * 8] = packed;
  }
  if (q_t == nullptr) return;
  __syncthreads();
  // Transposed copy: thread writes 16 consecutive source rows of one column.
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int idx = p * 256 + threadIdx.x;  // 1024 = 128 columns x 8 row groups
    const int c = idx >> 3, rg = idx & 7;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t)tile[rg * 16 + i][c] << (8 * (i & 3));
    const int tcol = bi * 128 + c, trow = bo * 128 + rg * 16;
    if (tcol < in && trow < out)
      store_stream(q_t + ebase + (size_t)tcol * out + trow, make_uint4(w[0], w[1], w[2], w[3]));
  }
}

// e4m3 [E,R,C] -> [E,C,R] through a 128x128 LDS tile.
__global__ void __launch_bounds__(256) transpose_fp8_kernel(const uint8_t* __restrict__ src,
                                                            int rows, int cols,
                                                            uint8_t* __restrict__ dst) {
  __shared__ uint8_t tile[128][128 + 8];
  const int e = blockIdx.z, br = blockIdx.y, bc = blockIdx.x;
  const size_t ebase = (size_t)e * rows * cols;
  const int lane8 = threadIdx.x & 7, rsub = threadIdx.x >> 3;  // 8 x 16B per 128B row
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int r = br * 128 + p * 32 + rsub, c = bc * 128 + lane8 * 16;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (r < rows && c < cols) val = *(const uint4*)(src + ebase + (size_t)r * cols + c);
    *(uint2*)&tile[p * 32 + rsub][lane8 * 16] = make_uint2(val.x, val.y);
    *(uint2*)&tile[p * 32 + rsub][lane8 * 16 + 8] = make_uint2(val.z, val.w);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int idx = p * 256 + threadIdx.x;
    const int c = idx >> 4, rg = idx & 15;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo |= (uint32_t)tile[rg * 8 + i][c] << (8 * i);
      hi |= (uint32_t)tile[rg * 8 + 4 + i][c] << (8 * i);
    }
    const int tr = bc * 128 + c, tc = br * 128 + rg * 8;
    if (tr < cols && tc < rows) *(uint2*)(dst + ebase + (size_t)tr * rows + tc) = make_uint2(lo, hi);
  }
}

// ---------------------------------------------------------------------------
// Rows already in routed order -> e4m3 with 1x128 scales [width/128][rows].
// gate_up: the source row is [g0,u0,g1,u1,...]; store gates then ups.
// row_scales: scales [rows][width/128] instead (a row's scales together: the
// gathered GEMM's per-step scale reads of a token then share one line).
__global__ void __launch_bounds__(256) quantize_rows_kernel(const uint16_t* __restrict__ x,
                                                            int rows, int width, int64_t pitch,
                                                            int gate_up, uint8_t* __restrict__ q,
                                                            float* __restrict__ scales,
                                                            int row_scales = 0) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;
  const uint16_t* src = x + (size_t)r * pitch;
  // Up to four 512-column chunks' loads are issued before any of their
  // stores: loads and stores share one completion counter, so a load issued
  // after a store would wait for it.
  constexpr int kChunks = 4;
  if (!gate_up) {
    for (int base0 = 0; base0 < width; base0 += 512 * kChunks) {
      uint4 raw[kChunks];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        const int col = base0 + c * 512 + lane * 8;
        raw[c] = col < width ? *(const uint4*)(src + col) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        if (base0 + c * 512 >= width) break;  // uniform over the wave
        const int col = base0 + c * 512 + lane * 8;
        float v[8];
        unpack_bf16x8(raw[c], v);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = group_amax<16>(amax);
        const float s = fmaxf(amax * kInv448, kMinScale);
        const uint2 packed = quant8(v, s);
        if (col < width) {
          store_stream8(q + (size_t)r * width + col, packed);
          if ((lane & 15) == 0) {
            const size_t si = row_scales ? (size_t)r * (width >> 7) + (col >> 7)
                                         : (size_t)(col >> 7) * rows + r;
            scales[si] = s;
          }
        }
      }
    }
    return;
  }
  const int half = width / 2;
  for (int base0 = 0; base0 < half; base0 += 512 * kChunks) {
    uint4 ra[kChunks], rb[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int j = base0 + c * 512 + lane * 8;  // gate/up pair index
      ra[c] = rb[c] = make_uint4(0, 0, 0, 0);
      if (j < half) {
        ra[c] = *(const uint4*)(src + 2 * j);
        rb[c] = *(const uint4*)(src + 2 * j + 8);
      }
    }
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (base0 + c * 512 >= half) break;  // uniform over the wave
      const int j = base0 + c * 512 + lane * 8;
      float a[8], b[8], g[8], u[8];
      unpack_bf16x8(ra[c], a);
      unpack_bf16x8(rb[c], b);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[i] = a[2 * i]; u[i] = a[2 * i + 1];
        g[4 + i] = b[2 * i]; u[4 + i] = b[2 * i + 1];
      }
      float ga = 0.0f, ua = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ga = fmaxf(ga, fabsf(g[i]));
        ua = fmaxf(ua, fabsf(u[i]));
      }
      ga = group_amax<16>(ga);
      ua = group_amax<16>(ua);
      const float sg = fmaxf(ga * kInv448, kMinScale), su = fmaxf(ua * kInv448, kMinScale);
      const uint2 pg = quant8(g, sg), pu = quant8(u, su);
      if (j < half) {
        store_stream8(q + (size_t)r * width + j, pg);
        store_stream8(q + (size_t)r * width + half + j, pu);
        if ((lane & 15) == 0) {
          scales[(size_t)(j >> 7) * rows + r] = sg;
          scales[(size_t)((half + j) >> 7) * rows + r] = su;
        }
      }
    }
  }
}


// SwiGLU of interleaved h [rows, 2I] -> e4m3 act [rows, I] + 1x128 scales.
// Unit of work = (row, 128-column act group), taken by a 16-lane group (8
// columns = 16 interleaved h values per lane); each group handles kSwUnits
// units with every load issued before any math (memory parallelism), and
// stores full 128-byte act lines.
constexpr int kSwUnits = 4;

// The kernel is ALU-bound (exp, reciprocal and a correctly rounded division
// per element), so the unit -> (row, group) split is done once per group of
// lanes in 32-bit arithmetic and then stepped, and the clamp is a template
// flag rather than a per-element select.
template <bool kClamp>
__global__ void __launch_bounds__(256) swiglu_quantize_kernel(const uint16_t* __restrict__ h,
                                                              int rows, int width, float limit,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ scales,
                                                              uint16_t* __restrict__ act_out) {
  const uint32_t groups = (uint32_t)width / 128u;
  const uint32_t units = (uint32_t)rows * groups;  // < 2^31, checked on the host
  const int lane16 = threadIdx.x & 15;
  const uint32_t g0 = (blockIdx.x * 16u + (threadIdx.x >> 4)) * (uint32_t)kSwUnits;
  const uint32_t r0 = g0 / groups;
  const uint32_t grp0 = g0 - r0 * groups;
  uint32_t urow[kSwUnits], ugrp[kSwUnits];
  {
    uint32_t r = r0, grp = grp0;
#pragma unroll
    for (int u = 0; u < kSwUnits; ++u) {
      urow[u] = r;
      ugrp[u] = grp;
      if (++grp == groups) { grp = 0; ++r; }
    }
  }
  // Unit g covers h elements [256 g, 256 g + 256) and act / q elements
  // [128 g, 128 g + 128): a row holds `groups` units back to back in both.
  const uint16_t* src = h + (size_t)g0 * 256 + lane16 * 16;
  const size_t dst0 = (size_t)g0 * 128 + lane16 * 8;
  uint4 ha[kSwUnits], hb[kSwUnits];
#pragma unroll
  for (int u = 0; u < kSwUnits; ++u) {
    ha[u] = hb[u] = make_uint4(0, 0, 0, 0);
    if (g0 + u < units) {
      ha[u] = load_stream(src + u * 256);
      hb[u] = load_stream(src + u * 256 + 8);
    }
  }
#pragma unroll
  for (int u = 0; u < kSwUnits; ++u) {
    if (g0 + u >= units) break;  // uniform over the 16-lane group
    float a[8], b[8], act[8];
    unpack_bf16x8(ha[u], a);
    unpack_bf16x8(hb[u], b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float g0v = a[2 * i], u0 = a[2 * i + 1], g1 = b[2 * i], u1 = b[2 * i + 1];
      if (kClamp) {
        clamp_gate_up(g0v, u0, limit);
        clamp_gate_up(g1, u1, limit);
      }
      act[i] = silu_f(g0v) * u0;
      act[4 + i] = silu_f(g1) * u1;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(act[i]));
    amax = group_amax<16>(amax);
    const float sc = fmaxf(amax * kInv448, kMinScale);
    store_stream8(q + dst0 + u * 128, quant8(act, sc));
    if (lane16 == 0) scales[(size_t)ugrp[u] * rows + urow[u]] = sc;
    if (act_out != nullptr) {
      uint4 o;
      o.x = pack_bf16x2(act[0], act[1]);
      o.y = pack_bf16x2(act[2], act[3]);
      o.z = pack_bf16x2(act[4], act[5]);
      o.w = pack_bf16x2(act[6], act[7]);
      store_stream(act_out + dst0 + u * 128, o);
    }
  }
}

// ---------------------------------------------------------------------------
// Weight-gradient operand: routed rows (optionally gathered) transposed to
// feature-major e4m3, each expert's rows at its 128-aligned padded offset.
// Block = (padded 128-row block, 128 source columns).
constexpr int kQtPitch = 128 + 8;  // bf16 per LDS row: 272 B keeps 16-byte row alignment

// Every thread of the block calls this (it holds barriers); `active` ones
// (t in [0, 256)) do the work. The bf16 tile [128 rows][128 columns] becomes
// 128 feature rows of the weight-gradient layout: thread (4 columns fg, 16
// rows rb) takes its values and column maxima (combined over the 8 row
// groups through pmax), quantizes with power-of-two scales and stages the
// bytes in LDS as [column][row] over the tile's own memory (every read of
// the tile is behind the first barrier); then 8 lanes per column write its
// 128 rows as one whole 128-byte line. Column lc is feature feat0 + lc, or,
// with gate_half > 0 (an interleaved gate/up source), source column c0 + lc
// -> gate (even) or up (odd) feature.
constexpr int kQtLine = 128 + 16;  // LDS bytes per staged feature row

__device__ __forceinline__ int tile_feature(int lc, int feat0, int c0, int gate_half) {
  if (gate_half == 0) return feat0 + lc;
  const int src = c0 + lc;
  return (src & 1) ? gate_half + (src >> 1) : (src >> 1);
}

__device__ __forceinline__ void transpose_tile_pow2(bool active, uint16_t* tile,
                                                    float (*pmax)[128], int t, uint8_t* qt,
                                                    float* scales, int feat0, int c0,
                                                    int gate_half, int width_f, int padded,
                                                    int pb) {
  const int fg = t & 31, rb = t >> 5;
  float v[16][4];
  float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (active) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint2 d = *(const uint2*)&tile[(rb * 16 + i) * kQtPitch + 4 * fg];
      v[i][0] = bf16_to_f32(d.x & 0xffff);
      v[i][1] = bf16_to_f32(d.x >> 16);
      v[i][2] = bf16_to_f32(d.y & 0xffff);
      v[i][3] = bf16_to_f32(d.y >> 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) m[j] = fmaxf(m[j], fabsf(v[i][j]));
    }
    *(float4*)&pmax[rb][4 * fg] = make_float4(m[0], m[1], m[2], m[3]);
  }
  __syncthreads();
  uint8_t* staged = reinterpret_cast<uint8_t*>(tile);
  if (active) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float4 q = *(const float4*)&pmax[r][4 * fg];
      m[0] = fmaxf(m[0], q.x);
      m[1] = fmaxf(m[1], q.y);
      m[2] = fmaxf(m[2], q.z);
      m[3] = fmaxf(m[3], q.w);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sc = pow2_ceil(fmaxf(m[j] * kInv448, kMinScale));
      // v / sc is exact (sc a power of two) and within +-448 (v bf16).
      uint4 w;
      w.x = f32x4_to_e4m3_pow2(v[0][j], v[1][j], v[2][j], v[3][j], sc);
      w.y = f32x4_to_e4m3_pow2(v[4][j], v[5][j], v[6][j], v[7][j], sc);
      w.z = f32x4_to_e4m3_pow2(v[8][j], v[9][j], v[10][j], v[11][j], sc);
      w.w = f32x4_to_e4m3_pow2(v[12][j], v[13][j], v[14][j], v[15][j], sc);
      *(uint4*)&staged[(4 * fg + j) * kQtLine + rb * 16] = w;
      if (rb == 0)
        scales[(size_t)pb * width_f + tile_feature(4 * fg + j, feat0, c0, gate_half)] = sc;
    }
  }
  __syncthreads();
  if (!active) return;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int lc = pass * 32 + (t >> 3), part = t & 7;
    const int feat = tile_feature(lc, feat0, c0, gate_half);
    store_stream(qt + (size_t)feat * padded + (size_t)pb * 128 + part * 16,
                 *(const uint4*)&staged[lc * kQtLine + part * 16]);
  }
}


__global__ void __launch_bounds__(256) quantize_transpose_kernel(
    const uint16_t* __restrict__ x, int64_t pitch, int width, const int32_t* __restrict__ gather,
    int gather_div, int gate_up, const int32_t* __restrict__ row_blocks, int padded,
    uint8_t* __restrict__ qt, float* __restrict__ scales) {
  __shared__ __align__(16) uint16_t tile[128 * kQtPitch];
  __shared__ __align__(16) float pmax[8][128];
  const int pb = blockIdx.x, cb = blockIdx.y, tid = threadIdx.x;
  const int r0 = row_blocks[2 * pb], nvalid = row_blocks[2 * pb + 1];
  if (nvalid <= 0) return;  // past the last expert's rows
  const int c0 = cb * 128;
  // 128 rows x 128 source columns (bf16) into LDS, zeros past the expert.
  {
    // All eight source rows first, then all eight row loads, then the LDS
    // stores: the row loads depend on the gather loads, and loads complete
    // in order, so interleaving them per row would hold each row's load
    // behind the previous row's data.
    const int lane16 = tid & 15, rsub = tid >> 4;
    int src[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int rr = p * 16 + rsub;
      src[p] = r0 + (rr < nvalid ? rr : 0);
      if (gather != nullptr && rr < nvalid) src[p] = gather[src[p]] / gather_div;
    }
    uint4 val[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int rr = p * 16 + rsub;
      val[p] = make_uint4(0, 0, 0, 0);
      if (rr < nvalid) val[p] = *(const uint4*)(x + (size_t)src[p] * pitch + c0 + lane16 * 8);
    }
#pragma unroll
    for (int p = 0; p < 8; ++p)
      *(uint4*)&tile[(p * 16 + rsub) * kQtPitch + lane16 * 8] = val[p];
  }
  __syncthreads();
  transpose_tile_pow2(true, tile, pmax, tid, qt, scales, c0, c0, gate_up ? width / 2 : 0, width,
                      padded, pb);
}

// ---------------------------------------------------------------------------
// Routed SwiGLU backward, one wave per sorted row.
// h and dh may be the same buffer (dh written in place over h): each lane
// loads its h values before it stores their gradients, and no other lane
// reads them, so they carry no __restrict__.
template <bool kClamp>
__global__ void __launch_bounds__(256) routed_swiglu_bwd_kernel(
    const uint16_t* __restrict__ rmat, const uint16_t* h,
    const float* __restrict__ weights, const int32_t* __restrict__ order, int rows, int width,
    float limit, uint16_t* dh, uint16_t* __restrict__ a_prime,
    float* __restrict__ dscore, uint8_t* __restrict__ dhq, float* __restrict__ dhs) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int row = blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const float score = weights[order[row]];
  const uint16_t* hr = h + (size_t)row * 2 * width;
  const uint16_t* rr = rmat + (size_t)row * width;
  // The score dot in swiglu_bwd_quantize_kernel's order: a lane's 8
  // products, summed over each 128-column block's 16 lanes, and the block
  // sums added in block order, so both kernels give the same dscore.
  float dsum = 0.0f;
  // Two 512-column chunks' loads are issued before either's stores (loads
  // and stores share one completion counter).
  for (int base0 = 0; base0 < width; base0 += 1024) {
    uint4 hv0[2], hv1[2], rv[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int j = base0 + c * 512 + lane * 8;
      hv0[c] = hv1[c] = rv[c] = make_uint4(0, 0, 0, 0);
      if (j < width) {
        hv0[c] = *(const uint4*)(hr + 2 * j);
        hv1[c] = *(const uint4*)(hr + 2 * j + 8);
        rv[c] = *(const uint4*)(rr + j);
      }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int base = base0 + c * 512;
      if (base >= width) break;  // uniform over the wave
      const int j = base + lane * 8;
      float dot = 0.0f;
      if (j < width) {
        float a[8], b[8], r[8];
        unpack_bf16x8(hv0[c], a);
        unpack_bf16x8(hv1[c], b);
        unpack_bf16x8(rv[c], r);
        float dg[8], du[8], ap[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float rg = i < 4 ? a[2 * i] : b[2 * (i - 4)];
          const float ru = i < 4 ? a[2 * i + 1] : b[2 * (i - 4) + 1];
          float gv = rg, uv = ru;
          if (kClamp) clamp_gate_up(gv, uv, limit);
          const float sig = sigmoid_f(gv);
          const float silu = gv * sig;
          const float act = silu * uv;
          dot += r[i] * act;
          const float gg = r[i] * score;
          float dgate = gg * uv * (sig + silu * (1.0f - sig));
          float dup = gg * silu;
          if (kClamp) {
            dgate = rg <= limit ? dgate : 0.0f;
            dup = (ru >= -limit && ru <= limit) ? dup : 0.0f;
          }
          dg[i] = dgate;
          du[i] = dup;
          ap[i] = act * score;
        }
        uint4 o0, o1, o2;
        o0.x = pack_bf16x2(dg[0], du[0]); o0.y = pack_bf16x2(dg[1], du[1]);
        o0.z = pack_bf16x2(dg[2], du[2]); o0.w = pack_bf16x2(dg[3], du[3]);
        o1.x = pack_bf16x2(dg[4], du[4]); o1.y = pack_bf16x2(dg[5], du[5]);
        o1.z = pack_bf16x2(dg[6], du[6]); o1.w = pack_bf16x2(dg[7], du[7]);
        o2.x = pack_bf16x2(ap[0], ap[1]); o2.y = pack_bf16x2(ap[2], ap[3]);
        o2.z = pack_bf16x2(ap[4], ap[5]); o2.w = pack_bf16x2(ap[6], ap[7]);
        *(uint4*)(dh + (size_t)row * 2 * width + 2 * j) = o0;
        *(uint4*)(dh + (size_t)row * 2 * width + 2 * j + 8) = o1;
        if (a_prime != nullptr) *(uint4*)(a_prime + (size_t)row * width + j) = o2;
        if (dhq != nullptr) {
          // dh row-quantized gate-first from its bf16 values, as the row
          // quantizer would read them back: the 16 lanes of this 128-column
          // block hold gate block j / 128 and up block I / 128 + j / 128
          // (width is a multiple of 128 here, so the group is all valid).
          const uint32_t w8[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
          float gq[8], uq[8];
          float ga = 0.0f, ua = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            gq[i] = bf16_to_f32(w8[i] & 0xffff);
            uq[i] = bf16_to_f32(w8[i] >> 16);
            ga = fmaxf(ga, fabsf(gq[i]));
            ua = fmaxf(ua, fabsf(uq[i]));
          }
          ga = group_amax<16>(ga);
          ua = group_amax<16>(ua);
          const float sg = fmaxf(ga * kInv448, kMinScale), su = fmaxf(ua * kInv448, kMinScale);
          uint8_t* qrow = dhq + (size_t)row * 2 * width;
          store_stream8(qrow + j, quant8(gq, sg));
          store_stream8(qrow + width + j, quant8(uq, su));
          if ((lane & 15) == 0) {
            dhs[(size_t)(j >> 7) * rows + row] = sg;
            dhs[(size_t)(width / 128 + (j >> 7)) * rows + row] = su;
          }
        }
      }
      dot = group_sum<16>(dot);
      const int blocks = min(4, (width - base + 127) / 128);  // 128-column blocks here
      for (int q = 0; q < blocks; ++q) dsum += __shfl(dot, 16 * q, 64);
    }
  }
  if (lane == 0) dscore[row] = dsum;
}


// ---------------------------------------------------------------------------
// Fused routed SwiGLU backward + every quantizer its outputs feed. Block =
// (padded 128-row block pb, 128 columns cb of I), 512 threads. Per block:
//  1. r [128 rows x 128 j] and the matching interleaved h are read once; dh
//     (gate, up) and a' are computed as in routed_swiglu_bwd_kernel and
//     rounded to bf16 (the values the unfused path stores);
//  2. dh rows are quantized 1x128 (gate block cb and up block I/128 + cb of
//     the gate-first layout) by 16-lane groups, straight from registers;
//  3. the per-row score dot over these 128 j goes to dsp[cb][row] (summed in
//     a fixed order by dscore_reduce_kernel);
//  4. the three bf16 tiles are staged in LDS (a' after dh) and written transposed (dh
//     features cb*128 + j and I + cb*128 + j, a' features cb*128 + j) with
//     power-of-two scales, as quantize_transpose_kernel does.
constexpr int kSbThreads = 512;

template <bool kClamp, bool kFull>
__device__ __forceinline__ void swiglu_bwd_block(
    const uint16_t* __restrict__ rmat, const uint16_t* __restrict__ h,
    const float* __restrict__ weights, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_blocks, int rows, int width, int padded, float limit,
    uint8_t* __restrict__ dhq, float* __restrict__ dhs, uint8_t* __restrict__ dht,
    float* __restrict__ dhts, uint8_t* __restrict__ apt, float* __restrict__ apts,
    float* __restrict__ dsp, uint16_t* __restrict__ dh,
    uint16_t (*tiles)[128 * kQtPitch], int cb, int r0, int nvalid, uint4* apk) {
  const int tid = threadIdx.x;

  // Phases 1-3: 16 lanes per row (8 j each), 32 rows per pass, 4 passes;
  // every pass's loads are issued before any compute (memory parallelism).
  const int lane16 = tid & 15, rsub = tid >> 4;
  const int jl = lane16 * 8, j = cb * 128 + jl;
  const int nblk = width / 128;
  uint4 hv0[4], hv1[4], rv4[4];
  float score[4];
  // The rows' order entries first: each score is a load that depends on
  // one, and loads complete in order, so an order load issued after a
  // pass's h and r loads would hold the next pass's loads back until they
  // land.
  int orow[4];
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int rr = pass * 32 + rsub;
    orow[pass] = (kFull || rr < nvalid) ? order[r0 + rr] : 0;
  }
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int rr = pass * 32 + rsub;
    hv0[pass] = hv1[pass] = rv4[pass] = make_uint4(0, 0, 0, 0);
    if (kFull || rr < nvalid) {
      const int row = r0 + rr;
      const uint16_t* hp = h + (size_t)row * 2 * width + 2 * j;
      hv0[pass] = *(const uint4*)hp;
      hv1[pass] = *(const uint4*)(hp + 8);
      rv4[pass] = *(const uint4*)(rmat + (size_t)row * width + j);
    }
  }
#pragma unroll
  for (int pass = 0; pass < 4; ++pass)
    score[pass] = (kFull || pass * 32 + rsub < nvalid) ? weights[orow[pass]] : 0.0f;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int rr = pass * 32 + rsub;
    const bool valid = (kFull || rr < nvalid);  // uniform over the 16-lane group
    uint4 og = make_uint4(0, 0, 0, 0), ou = og, oa = og;
    if (valid) {
      const int row = r0 + rr;
      float a[8], b[8], rv[8];
      unpack_bf16x8(hv0[pass], a);
      unpack_bf16x8(hv1[pass], b);
      unpack_bf16x8(rv4[pass], rv);
      float dg[8], du[8], ap[8], dot = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float rg = i < 4 ? a[2 * i] : b[2 * (i - 4)];
        const float ru = i < 4 ? a[2 * i + 1] : b[2 * (i - 4) + 1];
        float gv = rg, uv = ru;
        if (kClamp) clamp_gate_up(gv, uv, limit);
        const float sig = sigmoid_f(gv);
        const float silu = gv * sig;
        const float act = silu * uv;
        dot += rv[i] * act;
        const float gg = rv[i] * score[pass];
        float dgate = gg * uv * (sig + silu * (1.0f - sig));
        float dup = gg * silu;
        if (kClamp) {
          dgate = rg <= limit ? dgate : 0.0f;
          dup = (ru >= -limit && ru <= limit) ? dup : 0.0f;
        }
        dg[i] = dgate;
        du[i] = dup;
        ap[i] = act * score[pass];
      }
      og = make_uint4(pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3]),
                      pack_bf16x2(dg[4], dg[5]), pack_bf16x2(dg[6], dg[7]));
      ou = make_uint4(pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3]),
                      pack_bf16x2(du[4], du[5]), pack_bf16x2(du[6], du[7]));
      oa = make_uint4(pack_bf16x2(ap[0], ap[1]), pack_bf16x2(ap[2], ap[3]),
                      pack_bf16x2(ap[4], ap[5]), pack_bf16x2(ap[6], ap[7]));
      dot = group_sum<16>(dot);
      if (lane16 == 0) dsp[(size_t)cb * rows + row] = dot;
      if (dh != nullptr) {
        // bf16 dh in h's interleaved order (2j' = gate j', 2j' + 1 = up j').
        const uint32_t g4[4] = {og.x, og.y, og.z, og.w}, u4[4] = {ou.x, ou.y, ou.z, ou.w};
        uint32_t wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t gb = (g4[i >> 1] >> (16 * (i & 1))) & 0xffffu;
          const uint32_t ub = (u4[i >> 1] >> (16 * (i & 1))) & 0xffffu;
          wv[i] = gb | (ub << 16);
        }
        uint16_t* dp = dh + (size_t)row * 2 * width + 2 * j;
        *(uint4*)dp = make_uint4(wv[0], wv[1], wv[2], wv[3]);
        *(uint4*)(dp + 8) = make_uint4(wv[4], wv[5], wv[6], wv[7]);
      } else {
      // Row quantization of the bf16 values (gate-first 1x128 layout).
      float gq[8], uq[8];
      unpack_bf16x8(og, gq);
      unpack_bf16x8(ou, uq);
      float ga = 0.0f, ua = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ga = fmaxf(ga, fabsf(gq[i]));
        ua = fmaxf(ua, fabsf(uq[i]));
      }
      ga = group_amax<16>(ga);
      ua = group_amax<16>(ua);
      const float sg = fmaxf(ga * kInv448, kMinScale), su = fmaxf(ua * kInv448, kMinScale);
      // Streaming stores: the outputs are far larger than L2 and are read
      // back only by later launches.
      store_stream8(dhq + (size_t)row * 2 * width + j, quant8(gq, sg));
      store_stream8(dhq + (size_t)row * 2 * width + width + j, quant8(uq, su));
      if (lane16 == 0) {
        dhs[(size_t)cb * rows + row] = sg;
        dhs[(size_t)(nblk + cb) * rows + row] = su;
      }
      }
    }
    *(uint4*)&tiles[0][rr * kQtPitch + jl] = og;
    *(uint4*)&tiles[1][rr * kQtPitch + jl] = ou;
    apk[pass] = oa;
  }
}


// Four waves per SIMD (at most 128 registers): the two bodies below would
// otherwise be allocated 144, and the LDS already limits a CU to two blocks.
template <bool kClamp>
__global__ void __launch_bounds__(kSbThreads) __attribute__((amdgpu_waves_per_eu(4)))
swiglu_bwd_quantize_kernel(
    const uint16_t* __restrict__ rmat, const uint16_t* __restrict__ h,
    const float* __restrict__ weights, const int32_t* __restrict__ order,
    const int32_t* __restrict__ row_blocks, int rows, int width, int padded, float limit,
    uint8_t* __restrict__ dhq, float* __restrict__ dhs, uint8_t* __restrict__ dht,
    float* __restrict__ dhts, uint8_t* __restrict__ apt, float* __restrict__ apts,
    float* __restrict__ dsp, uint16_t* __restrict__ dh) {
  // dgate and dup tiles (a' is staged through tile 0 afterwards): ~74 KB,
  // two blocks per CU.
  __shared__ __align__(16) uint16_t tiles[2][128 * kQtPitch];
  __shared__ __align__(16) float pmax[2][8][128];
  const int pb = blockIdx.x, cb = blockIdx.y;
  const int r0 = row_blocks[2 * pb], nvalid = row_blocks[2 * pb + 1];
  if (nvalid <= 0) return;  // past the last expert's rows
  // A whole block of rows (all but each expert's last block) takes a body
  // with no per-row validity tests: no zeroed registers for absent rows and
  // no masked branches around their loads, arithmetic and stores.
  uint4 apk[4];  // this thread's packed bf16 a' (4 rows x 8 columns)
  if (nvalid >= 128)
    swiglu_bwd_block<kClamp, true>(rmat, h, weights, order, row_blocks, rows, width, padded,
                                   limit, dhq, dhs, dht, dhts, apt, apts, dsp, dh, tiles, cb,
                                   r0, nvalid, apk);
  else
    swiglu_bwd_block<kClamp, false>(rmat, h, weights, order, row_blocks, rows, width, padded,
                                    limit, dhq, dhs, dht, dhts, apt, apts, dsp, dh, tiles, cb,
                                    r0, nvalid, apk);
  // Phase 4 (both bodies): transposed outputs; threads 0-255 and 256-511
  // each take a tile.
  const int tid = threadIdx.x, rsub = tid >> 4, jl = (tid & 15) * 8;
  if (dht == nullptr && apt == nullptr) return;
  __syncthreads();
  const int half = tid >> 8, t = tid & 255;
  if (dht != nullptr)
    transpose_tile_pow2(true, tiles[half], pmax[half], t, dht, dhts, half * width + cb * 128,
                        0, 0, 2 * width, padded, pb);
  if (apt != nullptr) {
    __syncthreads();  // tile 0 and pmax[0] reuse
#pragma unroll
    for (int pass = 0; pass < 4; ++pass)
      *(uint4*)&tiles[0][(pass * 32 + rsub) * kQtPitch + jl] = apk[pass];
    __syncthreads();
    transpose_tile_pow2(half == 0, tiles[0], pmax[0], t, apt, apts, cb * 128, 0, 0, width,
                        padded, pb);
  }
}

__global__ void __launch_bounds__(256) dscore_reduce_kernel(const float* __restrict__ dsp,
                                                            int rows, int nblk,
                                                            float* __restrict__ dscore) {
  const int row = blockIdx.x * 256 + threadIdx.x;
  if (row >= rows) return;
  float s = 0.0f;
  for (int b = 0; b < nblk; ++b) s += dsp[(size_t)b * rows + row];
  dscore[row] = s;
}

// Padded 128-row block table of the weight-gradient layout: block pb ->
// (first sorted row, valid rows), valid = 0 past the last expert's blocks.
// Computed once per layout so the per-block kernels above need one load
// instead of an expert scan and search each.
__global__ void __launch_bounds__(1024) padded_row_blocks_kernel(
    const int32_t* __restrict__ offsets, int experts, int nblocks, int32_t* __restrict__ blocks) {
  __shared__ int ptile[1025];
  __shared__ int wsum[16];
  padded_block_prefix<1024>(offsets, experts, ptile, wsum);
  for (int pb = threadIdx.x; pb < nblocks; pb += 1024) {
    int r0 = 0, nvalid = 0;
    if (pb < ptile[experts]) {
      int lo = 0, hi = experts - 1;
      while (lo < hi) {  // last e with ptile[e] <= pb
        const int mid = (lo + hi + 1) >> 1;
        if (ptile[mid] <= pb) lo = mid; else hi = mid - 1;
      }
      r0 = offsets[lo] + (pb - ptile[lo]) * 128;
      nvalid = min(128, offsets[lo + 1] - r0);
    }
    blocks[2 * pb] = r0;
    blocks[2 * pb + 1] = nvalid;
  }
}

}  // namespace

extern "C" int mi355x_quantize_weight_blocks(const void* w, int is_fp32, int experts, int out,
                                             int in, uint8_t* q, float* scale, uint8_t* q_t,
                                             void* stream) {
  MI355X_REQUIRE(experts >= 0 && out > 0 && in > 0, "quantize_weight_blocks: bad shape");
  MI355X_REQUIRE(in % 16 == 0 && out % 16 == 0,
                 "quantize_weight_blocks: out and in must be multiples of 16");
  if (experts == 0) return MI355X_OK;
  const int bo = (out + 127) / 128, bi = (in + 127) / 128;
  dim3 grid(bi, bo, experts);
  if (is_fp32)
    hipLaunchKernelGGL(weight_blocks_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const float*)w, out, in, bo, bi, q, scale, q_t);
  else
    hipLaunchKernelGGL(weight_blocks_kernel<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)w, out, in, bo, bi, q, scale, q_t);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_transpose_fp8(const uint8_t* q, int experts, int rows, int cols,
                                    uint8_t* q_t, void* stream) {
  MI355X_REQUIRE(rows % 16 == 0 && cols % 16 == 0, "transpose_fp8: rows/cols must be multiples of 16");
  if (experts == 0 || rows == 0 || cols == 0) return MI355X_OK;
  dim3 grid((cols + 127) / 128, (rows + 127) / 128, experts);
  hipLaunchKernelGGL(transpose_fp8_kernel, grid, dim3(256), 0, (hipStream_t)stream, q, rows, cols,
                     q_t);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_quantize_rows_fp8(const void* x, int rows, int width, int64_t pitch,
                                        int gate_up, uint8_t* q, float* scales, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0, "quantize_rows: width must be a multiple of 128");
  MI355X_REQUIRE(!gate_up || width % 256 == 0,
                 "quantize_rows: a gate/up row needs halves that are multiples of 128");
  MI355X_REQUIRE(pitch >= width && pitch % 8 == 0, "quantize_rows: bad pitch");
  if (rows == 0) return MI355X_OK;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, rows, width, pitch, gate_up, q, scales);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_quantize_token_rows_fp8(const void* x, int rows, int width, uint8_t* q,
                                              float* scales, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0, "quantize_token_rows: width must be a multiple of 128");
  if (rows == 0) return MI355X_OK;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, rows, width, (int64_t)width, 0, q, scales, 1);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_swiglu_quantize_fp8(const void* h, int rows, int width, float limit,
                                          uint8_t* q, float* scales, void* act, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0, "swiglu_quantize: I must be a multiple of 128");
  if (rows == 0) return MI355X_OK;
  const long long units = (long long)rows * (width / 128);
  MI355X_REQUIRE(units < (1LL << 31), "swiglu_quantize: rows x I/128 must stay below 2^31");
  const long long blocks = (units + 16 * kSwUnits - 1) / (16 * kSwUnits);
  auto kernel = limit > 0.0f ? swiglu_quantize_kernel<true> : swiglu_quantize_kernel<false>;
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)h, rows, width, limit, q, scales, (uint16_t*)act);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" size_t mi355x_wgrad_padded_rows(int assignments, int experts) {
  size_t bound = (size_t)assignments + (size_t)experts * 127;
  return (bound + 127) / 128 * 128;
}

extern "C" int mi355x_padded_row_blocks(const int32_t* offsets, int experts, int padded,
                                        int32_t* blocks, void* stream) {
  MI355X_REQUIRE(experts > 0 && experts <= 1024, "padded_row_blocks: experts must be in [1, 1024]");
  MI355X_REQUIRE(padded >= 0 && padded % 128 == 0, "padded_row_blocks: padded must be a multiple of 128");
  if (padded == 0) return MI355X_OK;
  hipLaunchKernelGGL(padded_row_blocks_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream,
                     offsets, experts, padded / 128, blocks);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_quantize_transpose_fp8(const void* x, int64_t pitch, int width,
                                             const int32_t* gather, int gather_div, int gate_up,
                                             const int32_t* row_blocks, int padded, uint8_t* qt,
                                             float* scales, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0, "quantize_transpose: width must be a multiple of 128");
  MI355X_REQUIRE(!gate_up || width % 2 == 0, "quantize_transpose: gate/up width must be even");
  MI355X_REQUIRE(padded >= 0 && padded % 128 == 0, "quantize_transpose: padded must be a multiple of 128");
  MI355X_REQUIRE(gather == nullptr || gather_div > 0, "quantize_transpose: gather_div must be > 0");
  if (padded == 0) return MI355X_OK;
  dim3 grid(padded / 128, width / 128);
  hipLaunchKernelGGL(quantize_transpose_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, pitch, width, gather, gather_div, gate_up, row_blocks,
                     padded, qt, scales);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

namespace {
int routed_swiglu_launch(const void* r, const void* h, const float* weights, const int32_t* order,
                         int rows, int width, float limit, void* dh, void* a_prime, float* dscore,
                         uint8_t* dhq, float* dhs, void* stream) {
  if (rows == 0) return MI355X_OK;
  auto kernel = limit > 0.0f ? routed_swiglu_bwd_kernel<true> : routed_swiglu_bwd_kernel<false>;
  hipLaunchKernelGGL(kernel, dim3((rows + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)r, (const uint16_t*)h, weights, order,
                     rows, width, limit, (uint16_t*)dh, (uint16_t*)a_prime, dscore, dhq, dhs);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
}  // namespace

extern "C" int mi355x_routed_swiglu_bwd(const void* r, const void* h, const float* weights,
                                        const int32_t* order, int rows, int width, float limit,
                                        void* dh, void* a_prime, float* dscore, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0, "routed_swiglu_bwd: width must be a multiple of 8");
  return routed_swiglu_launch(r, h, weights, order, rows, width, limit, dh, a_prime, dscore,
                              nullptr, nullptr, stream);
}

extern "C" int mi355x_routed_swiglu_bwd_rows_fp8(const void* r, const void* h,
                                                 const float* weights, const int32_t* order,
                                                 int rows, int width, float limit, void* dh,
                                                 void* a_prime, float* dscore, uint8_t* dhq,
                                                 float* dh_scales, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0,
                 "routed_swiglu_bwd_rows_fp8: I must be a multiple of 128");
  MI355X_REQUIRE(dhq != nullptr && dh_scales != nullptr,
                 "routed_swiglu_bwd_rows_fp8: dhq and its scales are required");
  return routed_swiglu_launch(r, h, weights, order, rows, width, limit, dh, a_prime, dscore, dhq,
                              dh_scales, stream);
}

extern "C" size_t mi355x_swiglu_bwd_quantize_workspace_size(int rows, int width) {
  return (size_t)rows * (size_t)(width / 128) * sizeof(float);
}

namespace {
int swiglu_bwd_launch(const void* r, const void* h, const float* weights, const int32_t* order,
                      const int32_t* row_blocks, int rows, int width, int padded, float limit,
                      uint8_t* dhq, float* dh_scales, void* dh, uint8_t* dh_t, float* dh_t_scales,
                      uint8_t* ap_t, float* ap_t_scales, float* dscore, void* workspace,
                      size_t workspace_bytes, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 128 == 0, "swiglu_bwd_quantize: I must be a multiple of 128");
  MI355X_REQUIRE(padded >= 0 && padded % 128 == 0 && (size_t)padded >= (size_t)rows,
                 "swiglu_bwd_quantize: padded must be a multiple of 128 covering the rows");
  MI355X_REQUIRE((dh_t == nullptr) == (dh_t_scales == nullptr) &&
                     (ap_t == nullptr) == (ap_t_scales == nullptr),
                 "swiglu_bwd_quantize: transposed outputs need their scales");
  MI355X_REQUIRE(workspace_bytes >= mi355x_swiglu_bwd_quantize_workspace_size(rows, width),
                 "swiglu_bwd_quantize: workspace too small");
  if (rows == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  float* dsp = (float*)workspace;
  auto kernel = limit > 0.0f ? swiglu_bwd_quantize_kernel<true> : swiglu_bwd_quantize_kernel<false>;
  hipLaunchKernelGGL(kernel, dim3(padded / 128, width / 128), dim3(kSbThreads), 0, s, (const uint16_t*)r, (const uint16_t*)h, weights, order, row_blocks,
                     rows, width, padded, limit, dhq, dh_scales, dh_t, dh_t_scales, ap_t,
                     ap_t_scales, dsp, (uint16_t*)dh);
  MI355X_LAUNCH_CHECK();
  hipLaunchKernelGGL(dscore_reduce_kernel, dim3((rows + 255) / 256), dim3(256), 0, s, dsp, rows,
                     width / 128, dscore);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
}  // namespace

extern "C" int mi355x_swiglu_bwd_quantize(const void* r, const void* h, const float* weights,
                                          const int32_t* order, const int32_t* row_blocks,
                                          int rows, int width, int padded, float limit,
                                          uint8_t* dhq, float* dh_scales, uint8_t* dh_t,
                                          float* dh_t_scales, uint8_t* ap_t, float* ap_t_scales,
                                          float* dscore, void* workspace, size_t workspace_bytes,
                                          void* stream) {
  MI355X_REQUIRE(dhq != nullptr && dh_scales != nullptr, "swiglu_bwd_quantize: dhq is required");
  return swiglu_bwd_launch(r, h, weights, order, row_blocks, rows, width, padded, limit, dhq,
                           dh_scales, nullptr, dh_t, dh_t_scales, ap_t, ap_t_scales, dscore,
                           workspace, workspace_bytes, stream);
}

extern "C" int mi355x_swiglu_bwd_bf16(const void* r, const void* h, const float* weights,
                                      const int32_t* order, const int32_t* row_blocks, int rows,
                                      int width, int padded, float limit, void* dh, uint8_t* dh_t,
                                      float* dh_t_scales, uint8_t* ap_t, float* ap_t_scales,
                                      float* dscore, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  MI355X_REQUIRE(dh != nullptr, "swiglu_bwd_bf16: dh is required");
  return swiglu_bwd_launch(r, h, weights, order, row_blocks, rows, width, padded, limit, nullptr,
                           nullptr, dh, dh_t, dh_t_scales, ap_t, ap_t_scales, dscore, workspace,
                           workspace_bytes, stream);
}
