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
// Weights: read once per pass, through non-temporal loads.
template <typename T>
__device__ __forceinline__ void load8_once(const T* p, float* v) { load8(p, v); }
template <>
__device__ __forceinline__ void load8_once<uint16_t>(const uint16_t* p, float* v) {
  unpack_bf16x8(load_stream(p), v);
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
  amax = group_amax<64>(amax);
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
  amax = group_amax<64>(amax);
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
  amax = group_amax<64>(amax);
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
//  1. weight_amax_kernel: one block per (128 x 128 tile, expert), in the
//     tiling and thread layout of the quantize pass. It writes the tile's
//     maxima per stored row to rowpart[e][column tile][row] and per column
//     to colpart[e][row tile][column] in the workspace.
//  2. scale_reduce_kernel reduces the partials into the row scales and the
//     column scales (a maximum, so the order does not matter), and writes
//     each scale's reciprocal to the workspace for the quantize pass.
//  3. weight_quantize_kernel: one block per (128 x 128 tile, expert). It
//     quantizes the tile with its rows' scales into q, and with its columns'
//     scales into qt through an LDS transpose.
// Stored row p of an expert is logical row p, or with interleave the
// gate/up-adjacent order (2j = gate j, 2j + 1 = up j), in both orientations.
__device__ __forceinline__ int logical_row(int p, int out, int interleave) {
  return interleave ? ((p & 1) ? out / 2 + (p >> 1) : (p >> 1)) : p;
}

constexpr int kQTile = 128;

// Thread t of a 128 x 128 tile block holds the tile's stored rows
// rg * R + i (i < R) at the 8 columns cg * 8 + j, rg = t / 16, cg = t % 16:
// a wave's load instruction reads 4 rows x 256 contiguous bytes. All R
// loads are issued before any use.
template <int R, typename T>
__device__ __forceinline__ void load_tile(const T* __restrict__ we, int out, int in,
                                          int interleave, int p0, int col, int rg,
                                          float (&v)[R][8]) {
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int p = p0 + rg * R + i;
    if (p < out && col < in) {
      load8_once(we + (size_t)logical_row(p, out, interleave) * in + col, v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(512) weight_amax_kernel(
    const T* __restrict__ w, int out, int in, int interleave, float* __restrict__ rowpart,
    float* __restrict__ colpart) {
  __shared__ float colmax[8][kQTile];  // per-wave column maxima
  const int e = blockIdx.z, p0 = blockIdx.y * kQTile, c0 = blockIdx.x * kQTile;
  const int t = threadIdx.x, cg = t & 15, rg = t >> 4, wave = t >> 6;
  float v[4][8];
  load_tile<4>(w + (size_t)e * out * in, out, in, interleave, p0, c0 + cg * 8, rg, v);
  float rm[4], cm[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) cm[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rm[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = fabsf(v[i][j]);
      rm[i] = fmaxf(rm[i], a);
      cm[j] = fmaxf(cm[j], a);
    }
  }
  // Rows over the 16 column groups (lanes 16 apart share rows: xor 1..8);
  // columns over the wave's 4 row groups (xor 16, 32), then over the waves.
#pragma unroll
  for (int o = 1; o < 16; o <<= 1)
#pragma unroll
    for (int i = 0; i < 4; ++i) rm[i] = fmaxf(rm[i], __shfl_xor(rm[i], o, 64));
#pragma unroll
  for (int o = 16; o < 64; o <<= 1)
#pragma unroll
    for (int j = 0; j < 8; ++j) cm[j] = fmaxf(cm[j], __shfl_xor(cm[j], o, 64));
  const int p = p0 + rg * 4;
  if (cg == 0 && p < out)  // out % 16 == 0: all 4 rows exist
    *(float4*)(rowpart + ((size_t)e * gridDim.x + blockIdx.x) * out + p) =
        make_float4(rm[0], rm[1], rm[2], rm[3]);
  if ((t & 63) < 16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) colmax[wave][cg * 8 + j] = cm[j];
  }
  __syncthreads();
  if (t < kQTile && c0 + t < in) {
    float m = colmax[0][t];
#pragma unroll
    for (int k = 1; k < 8; ++k) m = fmaxf(m, colmax[k][t]);
    colpart[((size_t)e * gridDim.y + blockIdx.y) * in + c0 + t] = m;
  }
}

// Thread i < experts * out: row scale i from its ctiles partials; the next
// experts * in threads: column scale from its rtiles partials.
__global__ void __launch_bounds__(256) scale_reduce_kernel(
    const float* __restrict__ rowpart, const float* __restrict__ colpart, int experts, int out,
    int in, int ctiles, int rtiles, float* __restrict__ scales, float* __restrict__ scales_t,
    float* __restrict__ inverse) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t nrow = (size_t)experts * out;
  float m = 0.0f;
  if (i < nrow) {
    const size_t e = i / out, p = i - e * out;
    const float* part = rowpart + e * ctiles * out + p;
    for (int k = 0; k < ctiles; ++k) m = fmaxf(m, part[(size_t)k * out]);
    const float sc = fmaxf(m * kInv448, kMinScale);
    scales[i] = sc;
    inverse[i] = 1.0f / sc;
  } else if (i - nrow < (size_t)experts * in) {
    const size_t j = i - nrow, e = j / in, c = j - e * in;
    const float* part = colpart + e * rtiles * in + c;
    for (int k = 0; k < rtiles; ++k) m = fmaxf(m, part[(size_t)k * in]);
    const float sc = fmaxf(m * kInv448, kMinScale);
    scales_t[j] = sc;
    inverse[i] = 1.0f / sc;
  }
}

// 512 threads, 4 rows x 8 columns each: the two quantizations of every
// element (row scale for q, column scale for qt) make this pass ALU-heavy,
// and the small per-thread tile keeps ~8 waves per SIMD to hide the loads.
template <typename T>
__global__ void __launch_bounds__(512) weight_quantize_kernel(
    const T* __restrict__ w, int out, int in, int interleave, const float* __restrict__ scales,
    const float* __restrict__ scales_t, const float* __restrict__ inverse, uint8_t* __restrict__ q,
    uint8_t* __restrict__ qt) {
  __shared__ uint8_t tile[kQTile][kQTile + 8];  // [column][stored row]
  __shared__ float colscale[2][kQTile];         // column scales and their reciprocals
  const int e = blockIdx.z, p0 = blockIdx.y * kQTile, c0 = blockIdx.x * kQTile;
  const int t = threadIdx.x, cg = t & 15, rg = t >> 4;  // 16 column groups x 32 row groups
  const int col = c0 + cg * 8;
  const bool col_ok = col < in;
  float v[4][8];
  load_tile<4>(w + (size_t)e * out * in, out, in, interleave, p0, col, rg, v);
  // The row scales and the column scales are loaded before any store:
  // loads and stores complete in order, so a load behind a store waits.
  const int pr = min(p0 + rg * 4, out - 4);  // out % 16 == 0
  const float4 rs = *(const float4*)(scales + (size_t)e * out + pr);
  const float4 ri = *(const float4*)(inverse + (size_t)e * out + pr);
  if (t < 2 * kQTile) {
    const int c = t & (kQTile - 1);
    const float* src = t < kQTile ? scales_t + (size_t)e * in
                                  : inverse + (size_t)gridDim.z * out + (size_t)e * in;
    colscale[t >> 7][c] = c0 + c < in ? src[c0 + c] : 1.0f;
  }
  __syncthreads();
  const float rsv[4] = {rs.x, rs.y, rs.z, rs.w}, riv[4] = {ri.x, ri.y, ri.z, ri.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = p0 + rg * 4 + i;
    if (p < out && col_ok)
      *(uint2*)(q + ((size_t)e * out + p) * in + col) = quant8(v[i], rsv[i], riv[i]);
  }
  // Column j's bytes of the thread's 4 rows, one conversion pair each.
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float cs = colscale[0][cg * 8 + j], ci = colscale[1][cg * 8 + j];
    *(uint32_t*)&tile[cg * 8 + j][rg * 4] =
        f32x4_to_e4m3(quant_div_inv(v[0][j], cs, ci), quant_div_inv(v[1][j], cs, ci),
                      quant_div_inv(v[2][j], cs, ci), quant_div_inv(v[3][j], cs, ci));
  }
  __syncthreads();
  // 128 qt rows x 128 bytes, two passes of 64 rows: thread t writes 16 bytes.
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int cc = pass * 64 + (t >> 3), seg = (t & 7) * 16;
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
  const size_t rtiles = (out + kQTile - 1) / kQTile, ctiles = (in + kQTile - 1) / kQTile;
  return (size_t)experts * (ctiles * out + rtiles * in + out + in) * sizeof(float);
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
  const dim3 tile_grid((in + kQTile - 1) / kQTile, (out + kQTile - 1) / kQTile, experts);
  float* rowpart = (float*)workspace;
  float* colpart = rowpart + (size_t)experts * tile_grid.x * out;
  // Reciprocals of the row scales [E, out], then of the column scales [E, in].
  float* inverse = colpart + (size_t)experts * tile_grid.y * in;
  if (is_fp32) {
    hipLaunchKernelGGL(weight_amax_kernel<float>, tile_grid, dim3(512), 0, s, (const float*)w,
                       out, in, interleave, rowpart, colpart);
  } else {
    hipLaunchKernelGGL(weight_amax_kernel<uint16_t>, tile_grid, dim3(512), 0, s,
                       (const uint16_t*)w, out, in, interleave, rowpart, colpart);
  }
  const size_t n = (size_t)experts * (out + in);
  hipLaunchKernelGGL(scale_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     rowpart, colpart, experts, out, in, (int)tile_grid.x, (int)tile_grid.y,
                     scales, scales_t, inverse);
  if (is_fp32) {
    hipLaunchKernelGGL(weight_quantize_kernel<float>, tile_grid, dim3(512), 0, s, (const float*)w,
                       out, in, interleave, scales, scales_t, inverse, q, qt);
  } else {
    hipLaunchKernelGGL(weight_quantize_kernel<uint16_t>, tile_grid, dim3(512), 0, s,
                       (const uint16_t*)w, out, in, interleave, scales, scales_t, inverse, q, qt);
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
