// Current (per-row) e4m3 scaling of the "fp8_current" expert format: one
// descale per row of an operand, over its whole K extent, instead of 1x128 /
// 128x128 blocks. Equations of the reference's row quantizer
// (kernels/quack_moe/quantize_rows.py:35-41): scale = max(amax * (1/448),
// 1e-12) with the fp32-rounded reciprocal, q = e4m3(clip(x / scale, +-448))
// with a correctly rounded division.
//
// The kernels are HBM-bound. A row kernel reads its row twice, once for the
// maximum and once to quantize it; the second read hits the caches. Widths
// reach 28672 (Mixtral's gate/up rows), too wide to hold in registers.
#include "common.h"

namespace {

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* v) {
  load_bf16x8(p, v);
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* v) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Source row of stored row r: a gathered routed row (gather[r] / div, the
// token of a sorted assignment), a weight row in gate/up-adjacent order
// (stored row 2j of an expert = gate row j, 2j + 1 = up row j; interleave =
// the expert's row count), or r itself.
__device__ __forceinline__ long long source_row(int r, const int32_t* __restrict__ gather,
                                                int div, int interleave) {
  if (gather != nullptr) return gather[r] / div;
  if (interleave > 0) {
    const int e = r / interleave, p = r - e * interleave;
    return (long long)e * interleave + ((p & 1) ? interleave / 2 + (p >> 1) : (p >> 1));
  }
  return r;
}

// One wave per stored row, 8 columns per lane per 512-column pass.
template <typename T>
__global__ void __launch_bounds__(256) rows_current_kernel(
    const T* __restrict__ x, int rows, int width, int64_t pitch,
    const int32_t* __restrict__ gather, int div, int interleave, uint8_t* __restrict__ q,
    float* __restrict__ scales) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;
  const T* src = x + source_row(r, gather, div, interleave) * pitch;
  float amax = 0.0f;
  for (int col = lane * 8; col < width; col += 512) {
    float v[8];
    load8(src + col, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax * kInv448, kMinScale);
  uint8_t* dst = q + (size_t)r * width;
  // Four chunks' loads before their stores: loads and stores complete in
  // order, so a load issued after a store would wait for it.
  for (int col0 = lane * 8; col0 < width; col0 += 4 * 512) {
    float v[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col0 + c * 512 < width) load8(src + col0 + c * 512, v[c]);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col0 + c * 512 < width) *(uint2*)(dst + col0 + c * 512) = quant8(v[c], s);
  }
  if (lane == 0) scales[r] = s;
}

// Token-major form for routed copies of token rows (x, dy): one wave per
// token reads its row once, and writes the quantized row and its scale to
// each of the token's top_k sorted slots. A routed row's quantization
// depends only on its token's row, so this equals quantizing the gathered
// rows.
__global__ void __launch_bounds__(256) permute_rows_current_kernel(
    const uint16_t* __restrict__ x, int tokens, int width, int top_k,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ q, float* __restrict__ scales) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int t = blockIdx.x * 4 + wave;
  if (t >= tokens) return;
  const uint16_t* src = x + (size_t)t * width;
  float amax = 0.0f;
  for (int col = lane * 8; col < width; col += 512) {
    float v[8];
    load_bf16x8(src + col, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax * kInv448, kMinScale);
  // The token's slots in registers (read before any store), then four
  // chunks' loads before their stores.
  int dest[32];
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < top_k) dest[j] = slots[(size_t)t * top_k + j];
  for (int col0 = lane * 8; col0 < width; col0 += 4 * 512) {
    float v[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col0 + c * 512 < width) load_bf16x8(src + col0 + c * 512, v[c]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (col0 + c * 512 >= width) break;
      const uint2 packed = quant8(v[c], s);
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (j < top_k) *(uint2*)(q + (size_t)dest[j] * width + col0 + c * 512) = packed;
    }
  }
#pragma unroll
  for (int j = 0; j < 32; ++j)
    if (j < top_k && lane == j) scales[dest[j]] = s;
}

// SwiGLU of an interleaved pre-activation row h [2I] (clamped at limit when
// limit > 0), quantized per row: the down projection's operand. The
// activation is computed twice (for the maximum, then to quantize), as
// swiglu_quantize_kernel computes it.
__device__ __forceinline__ void swiglu8(const uint16_t* p, float limit, float* act) {
  float a[8], b[8];
  load_bf16x8(p, a);
  load_bf16x8(p + 8, b);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float g0 = a[2 * i], u0 = a[2 * i + 1], g1 = b[2 * i], u1 = b[2 * i + 1];
    clamp_gate_up(g0, u0, limit);
    clamp_gate_up(g1, u1, limit);
    act[i] = silu_f(g0) * u0;
    act[4 + i] = silu_f(g1) * u1;
  }
}

__global__ void __launch_bounds__(256) swiglu_rows_current_kernel(
    const uint16_t* __restrict__ h, int rows, int width, float limit, uint8_t* __restrict__ q,
    float* __restrict__ scales, uint16_t* __restrict__ act_out) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;
  const uint16_t* src = h + (size_t)r * 2 * width;
  float amax = 0.0f;
  for (int j = lane * 8; j < width; j += 512) {
    float act[8];
    swiglu8(src + 2 * j, limit, act);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(act[i]));
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax * kInv448, kMinScale);
  uint8_t* dst = q + (size_t)r * width;
  // Four chunks' loads before their stores (loads and stores complete in
  // order).
  for (int j0 = lane * 8; j0 < width; j0 += 4 * 512) {
    uint4 hv[4][2];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      hv[c][0] = hv[c][1] = make_uint4(0, 0, 0, 0);
      if (j0 + c * 512 < width) {
        hv[c][0] = *(const uint4*)(src + 2 * (j0 + c * 512));
        hv[c][1] = *(const uint4*)(src + 2 * (j0 + c * 512) + 8);
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j = j0 + c * 512;
      if (j >= width) break;
      float a[8], b[8], act[8];
      unpack_bf16x8(hv[c][0], a);
      unpack_bf16x8(hv[c][1], b);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float g0 = a[2 * i], u0 = a[2 * i + 1], g1 = b[2 * i], u1 = b[2 * i + 1];
        clamp_gate_up(g0, u0, limit);
        clamp_gate_up(g1, u1, limit);
        act[i] = silu_f(g0) * u0;
        act[4 + i] = silu_f(g1) * u1;
      }
      *(uint2*)(dst + j) = quant8(act, s);
      if (act_out != nullptr)  // the bf16 activation too (expert LoRA's down-projection term)
        *(uint4*)(act_out + (size_t)r * width + j) =
            make_uint4(pack_bf16x2(act[0], act[1]), pack_bf16x2(act[2], act[3]),
                       pack_bf16x2(act[4], act[5]), pack_bf16x2(act[6], act[7]));
    }
  }
  if (lane == 0) scales[r] = s;
}

// Both orientations of weights w [E, out, in] in two passes over w:
//  1. weight_amax_kernel: one block per (64 stored rows, expert). It writes
//     each row's scale (a wave reduces a whole row), and the maxima of its
//     rows per column to colpart[e][tile][c] in the workspace.
//  2. col_scale_kernel reduces colpart over the row tiles into the column
//     scales.
//  3. weight_quantize_kernel: one block per (128 x 128 tile, expert). It
//     quantizes the tile with its rows' scales into q, and with its columns'
//     scales into qt through an LDS transpose.
// Stored row p of an expert is logical row p, or with interleave the
// gate/up-adjacent order (2j = gate j, 2j + 1 = up j), in both orientations.
__device__ __forceinline__ int logical_row(int p, int out, int interleave) {
  return interleave ? ((p & 1) ? out / 2 + (p >> 1) : (p >> 1)) : p;
}

constexpr int kAmaxRows = 64;  // 3 x 256 blocks fill the GPU evenly for E = 128, out = 1536
constexpr int kQTile = 128;

template <typename T>
__global__ void __launch_bounds__(256) weight_amax_kernel(
    const T* __restrict__ w, int out, int in, int interleave, float* __restrict__ scales,
    float* __restrict__ colpart) {
  __shared__ float colmax[4][2048 + 8];  // per-wave column maxima of a 2048-column chunk
  const int e = blockIdx.y, tile = blockIdx.x, p0 = tile * kAmaxRows;
  const int tiles = gridDim.x;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const T* we = w + (size_t)e * out * in;
  const int prows = min(kAmaxRows, out - p0);
  for (int c0 = 0; c0 < in; c0 += 2048) {
    const int cw = min(2048, in - c0);
    float cm[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) cm[i] = 0.0f;
    // Wave w takes rows w, w + 4, ..., two at a time (all eight loads of a
    // pair issued before the maxima); lane l takes 8 columns per 512.
    for (int pr = wave; pr < prows; pr += 8) {
      float rmax[2] = {0.0f, 0.0f};
      float v[2][4][8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int p = p0 + pr + 4 * h;
        const T* row = we + (size_t)logical_row(p, out, interleave) * in + c0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int col = u * 512 + lane * 8;
          if (pr + 4 * h < prows && col < cw) {
            load8(row + col, v[h][u]);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[h][u][i] = 0.0f;
          }
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float a = fabsf(v[h][u][i]);
            rmax[h] = fmaxf(rmax[h], a);
            cm[u * 8 + i] = fmaxf(cm[u * 8 + i], a);
          }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float m_row = wave_max(rmax[h]);
        // The row's running maximum over the column chunks lives in scales[]
        // (this block is the row's only writer), finished after the last chunk.
        if (lane == 0 && pr + 4 * h < prows) {
          const size_t at = (size_t)e * out + p0 + pr + 4 * h;
          const float prev = c0 == 0 ? 0.0f : scales[at];
          const float m = fmaxf(prev, m_row);
          scales[at] = c0 + 2048 >= in ? fmaxf(m * kInv448, kMinScale) : m;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) colmax[wave][u * 512 + lane * 8 + i] = cm[u * 8 + i];
    __syncthreads();
    float* part = colpart + ((size_t)e * tiles + tile) * in + c0;
    for (int c = threadIdx.x; c < cw; c += 256)
      part[c] = fmaxf(fmaxf(colmax[0][c], colmax[1][c]), fmaxf(colmax[2][c], colmax[3][c]));
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256) col_scale_kernel(const float* __restrict__ colpart,
                                                        int experts, int tiles, int in,
                                                        float* __restrict__ scales_t) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // e * in + c
  if (i >= (size_t)experts * in) return;
  const size_t e = i / in, c = i - e * in;
  const float* part = colpart + e * tiles * in + c;
  float m = 0.0f;
  for (int k = 0; k < tiles; ++k) m = fmaxf(m, part[(size_t)k * in]);
  scales_t[i] = fmaxf(m * kInv448, kMinScale);
}

template <typename T>
__global__ void __launch_bounds__(256) weight_quantize_kernel(
    const T* __restrict__ w, int out, int in, int interleave, const float* __restrict__ scales,
    const float* __restrict__ scales_t, uint8_t* __restrict__ q, uint8_t* __restrict__ qt) {
  __shared__ uint8_t tile[kQTile][kQTile + 8];  // [column][stored row]
  __shared__ float colscale[kQTile];
  const int e = blockIdx.z, p0 = blockIdx.y * kQTile, c0 = blockIdx.x * kQTile;
  const int t = threadIdx.x, cg = t & 15, rg = t >> 4;  // 16 column groups x 16 row groups
  const int col = c0 + cg * 8;
  const bool col_ok = col < in;
  const T* we = w + (size_t)e * out * in;
  // The thread's 8 consecutive rows rg * 8 + i, all loads issued first.
  float v[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int p = p0 + rg * 8 + i;
    if (p < out && col_ok) {
      load8(we + (size_t)logical_row(p, out, interleave) * in + col, v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
    }
  }
  if (t < kQTile) colscale[t] = c0 + t < in ? scales_t[(size_t)e * in + c0 + t] : 1.0f;
  __syncthreads();
  float cs[8], ci[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    cs[j] = colscale[cg * 8 + j];
    ci[j] = 1.0f / cs[j];
  }
  uint32_t lo[8], hi[8];  // column j's bytes of the thread's 8 rows
#pragma unroll
  for (int j = 0; j < 8; ++j) lo[j] = hi[j] = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int p = p0 + rg * 8 + i;
    if (p < out && col_ok)
      *(uint2*)(q + ((size_t)e * out + p) * in + col) = quant8(v[i], scales[(size_t)e * out + p]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t b = f32x2_to_e4m3(quant_div_inv(v[i][j], cs[j], ci[j]), 0.0f) & 0xffu;
      if (i < 4) lo[j] |= b << (8 * i);
      else hi[j] |= b << (8 * (i - 4));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) *(uint2*)&tile[cg * 8 + j][rg * 8] = make_uint2(lo[j], hi[j]);
  __syncthreads();
  // 128 qt rows x 128 bytes, four passes of 32 rows: thread t writes 16 bytes.
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int cc = pass * 32 + (t >> 3), seg = (t & 7) * 16;
    if (c0 + cc < in && p0 + seg < out) {
      const uint2 a = *(const uint2*)&tile[cc][seg], b = *(const uint2*)&tile[cc][seg + 8];
      *(uint4*)(qt + ((size_t)e * in + c0 + cc) * out + p0 + seg) = make_uint4(a.x, a.y, b.x, b.y);
    }
  }
}

}  // namespace

extern "C" int mi355x_quantize_rows_current_fp8(const void* x, int rows, int width,
                                                int64_t pitch, const int32_t* gather,
                                                int gather_div, uint8_t* q, float* scales,
                                                void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0, "quantize_rows_current: width must be a multiple of 8");
  MI355X_REQUIRE(pitch >= width && pitch % 8 == 0, "quantize_rows_current: bad pitch");
  MI355X_REQUIRE(gather == nullptr || gather_div > 0, "quantize_rows_current: bad gather divisor");
  MI355X_REQUIRE(rows >= 0, "quantize_rows_current: negative rows");
  if (rows == 0) return MI355X_OK;
  hipLaunchKernelGGL(rows_current_kernel<uint16_t>, dim3((rows + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x, rows, width, pitch, gather,
                     gather_div, 0, q, scales);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_swiglu_quantize_rows_current_fp8(const void* h, int rows, int width,
                                                       float limit, uint8_t* q, float* scales,
                                                       void* act, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0,
                 "swiglu_quantize_rows_current: I must be a multiple of 8");
  MI355X_REQUIRE(rows >= 0, "swiglu_quantize_rows_current: negative rows");
  if (rows == 0) return MI355X_OK;
  hipLaunchKernelGGL(swiglu_rows_current_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)h, rows, width, limit, q, scales,
                     (uint16_t*)act);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" size_t mi355x_quantize_weights_current_workspace_size(int experts, int out, int in) {
  if (experts <= 0 || out <= 0 || in <= 0) return 0;
  return (size_t)experts * ((out + kAmaxRows - 1) / kAmaxRows) * in * sizeof(float);
}

extern "C" int mi355x_quantize_weights_current_fp8(const void* w, int is_fp32, int experts,
                                                   int out, int in, int interleave, uint8_t* q,
                                                   float* scales, uint8_t* qt, float* scales_t,
                                                   void* workspace, size_t workspace_bytes,
                                                   void* stream) {
  MI355X_REQUIRE(experts > 0 && out > 0 && in > 0, "quantize_weights_current: empty weight");
  MI355X_REQUIRE(in % 8 == 0, "quantize_weights_current: in must be a multiple of 8");
  MI355X_REQUIRE(out % 16 == 0, "quantize_weights_current: out must be a multiple of 16");
  MI355X_REQUIRE(workspace != nullptr &&
                     workspace_bytes >= mi355x_quantize_weights_current_workspace_size(experts, out, in),
                 "quantize_weights_current: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const int tiles = (out + kAmaxRows - 1) / kAmaxRows;
  float* colpart = (float*)workspace;
  const dim3 amax_grid(tiles, experts);
  const dim3 tile_grid((in + kQTile - 1) / kQTile, (out + kQTile - 1) / kQTile, experts);
  if (is_fp32) {
    hipLaunchKernelGGL(weight_amax_kernel<float>, amax_grid, dim3(256), 0, s, (const float*)w,
                       out, in, interleave, scales, colpart);
  } else {
    hipLaunchKernelGGL(weight_amax_kernel<uint16_t>, amax_grid, dim3(256), 0, s,
                       (const uint16_t*)w, out, in, interleave, scales, colpart);
  }
  const size_t ncol = (size_t)experts * in;
  hipLaunchKernelGGL(col_scale_kernel, dim3((unsigned)((ncol + 255) / 256)), dim3(256), 0, s,
                     colpart, experts, tiles, in, scales_t);
  if (is_fp32) {
    hipLaunchKernelGGL(weight_quantize_kernel<float>, tile_grid, dim3(256), 0, s, (const float*)w,
                       out, in, interleave, scales, scales_t, q, qt);
  } else {
    hipLaunchKernelGGL(weight_quantize_kernel<uint16_t>, tile_grid, dim3(256), 0, s,
                       (const uint16_t*)w, out, in, interleave, scales, scales_t, q, qt);
  }
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_permute_quantize_current_fp8(const void* x, int tokens, int width,
                                                   int top_k, const int32_t* slots, uint8_t* q,
                                                   float* scales, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0,
                 "permute_quantize_current: width must be a multiple of 8");
  MI355X_REQUIRE(top_k > 0 && top_k <= 32, "permute_quantize_current: top_k must be in [1, 32]");
  MI355X_REQUIRE(tokens >= 0, "permute_quantize_current: negative tokens");
  if (tokens == 0) return MI355X_OK;
  hipLaunchKernelGGL(permute_rows_current_kernel, dim3((tokens + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x, tokens, width, top_k, slots, q,
                     scales);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
