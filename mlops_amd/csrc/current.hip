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
  for (int col = lane * 8; col < width; col += 512) {
    float v[8];
    load8(src + col, v);
    *(uint2*)(dst + col) = quant8(v, s);
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
  const int32_t* dest = slots + (size_t)t * top_k;
  for (int col = lane * 8; col < width; col += 512) {
    float v[8];
    load_bf16x8(src + col, v);
    const uint2 packed = quant8(v, s);
    for (int j = 0; j < top_k; ++j) *(uint2*)(q + (size_t)dest[j] * width + col) = packed;
  }
  if (lane < top_k) scales[dest[lane]] = s;
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
    float* __restrict__ scales) {
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
  for (int j = lane * 8; j < width; j += 512) {
    float act[8];
    swiglu8(src + 2 * j, limit, act);
    *(uint2*)(dst + j) = quant8(act, s);
  }
  if (lane == 0) scales[r] = s;
}

// Both orientations of weights w [E, out, in] in two passes over w:
//  1. weight_amax_kernel: one block per (128 stored rows, expert). It writes
//     each row's scale (a wave reduces a whole row), and merges the rows'
//     column maxima into col_bits[e, c] with an integer atomicMax on the
//     float bits. Maxima are >= 0, so unsigned order is float order, and the
//     merge is order-independent.
//  2. weight_quantize_kernel: one block per (64 x 64 tile, expert). It
//     quantizes the tile with its rows' scales into q, and with its columns'
//     scales (from col_bits) into qt, through an LDS transpose.
//  3. col_scale_kernel turns col_bits into the column scales in place.
// Stored row p of an expert is logical row p, or with interleave the
// gate/up-adjacent order (2j = gate j, 2j + 1 = up j), in both orientations.
__device__ __forceinline__ int logical_row(int p, int out, int interleave) {
  return interleave ? ((p & 1) ? out / 2 + (p >> 1) : (p >> 1)) : p;
}

constexpr int kAmaxRows = 128;

template <typename T>
__global__ void __launch_bounds__(256) weight_amax_kernel(
    const T* __restrict__ w, int out, int in, int interleave, float* __restrict__ scales,
    uint32_t* __restrict__ col_bits) {
  __shared__ float colmax[4][2048 + 8];  // per-wave column maxima of a 2048-column chunk
  const int e = blockIdx.y, p0 = blockIdx.x * kAmaxRows;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const T* we = w + (size_t)e * out * in;
  const int prows = min(kAmaxRows, out - p0);
  for (int c0 = 0; c0 < in; c0 += 2048) {
    const int cw = min(2048, in - c0);
    float cm[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) cm[i] = 0.0f;
    // Wave w takes rows w, w + 4, ...; lane l takes 8 columns per 512.
    for (int pr = wave; pr < prows; pr += 4) {
      const int p = p0 + pr;
      const T* row = we + (size_t)logical_row(p, out, interleave) * in + c0;
      float rmax = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int col = u * 512 + lane * 8;
        if (col < cw) {
          float v[8];
          load8(row + col, v);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float a = fabsf(v[i]);
            rmax = fmaxf(rmax, a);
            cm[u * 8 + i] = fmaxf(cm[u * 8 + i], a);
          }
        }
      }
      rmax = wave_max(rmax);
      // The row's running maximum over the column chunks lives in scales[]
      // (this block is the row's only writer), finished after the last chunk.
      if (lane == 0) {
        const size_t at = (size_t)e * out + p;
        const float prev = c0 == 0 ? 0.0f : scales[at];
        const float m = fmaxf(prev, rmax);
        scales[at] = c0 + 2048 >= in ? fmaxf(m * kInv448, kMinScale) : m;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) colmax[wave][u * 512 + lane * 8 + i] = cm[u * 8 + i];
    __syncthreads();
    for (int c = threadIdx.x; c < cw; c += 256) {
      const float m = fmaxf(fmaxf(colmax[0][c], colmax[1][c]), fmaxf(colmax[2][c], colmax[3][c]));
      atomicMax(&col_bits[(size_t)e * in + c0 + c], __float_as_uint(m));
    }
    __syncthreads();
  }
}

constexpr int kQTile = 64;

template <typename T>
__global__ void __launch_bounds__(256) weight_quantize_kernel(
    const T* __restrict__ w, int out, int in, int interleave, const float* __restrict__ scales,
    const uint32_t* __restrict__ col_bits, uint8_t* __restrict__ q, uint8_t* __restrict__ qt) {
  __shared__ uint8_t tile[kQTile][kQTile + 16];  // [column][stored row]
  const int e = blockIdx.z, p0 = blockIdx.y * kQTile, c0 = blockIdx.x * kQTile;
  const int t = threadIdx.x, cg = t & 7, rl = t >> 3;  // 8 column groups x 32 rows
  const int col = c0 + cg * 8;
  const T* we = w + (size_t)e * out * in;
  float cs[8], ci[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float amax = col + i < in ? __uint_as_float(col_bits[(size_t)e * in + col + i]) : 0.0f;
    cs[i] = fmaxf(amax * kInv448, kMinScale);
    ci[i] = 1.0f / cs[i];
  }
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int pl = rl + 32 * half, p = p0 + pl;
    if (p < out && col < in) {
      float v[8];
      load8(we + (size_t)logical_row(p, out, interleave) * in + col, v);
      const float rs = scales[(size_t)e * out + p];
      *(uint2*)(q + ((size_t)e * out + p) * in + col) = quant8(v, rs);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        tile[cg * 8 + i][pl] =
            (uint8_t)(f32x2_to_e4m3(quant_div_inv(v[i], cs[i], ci[i]), 0.0f) & 0xffu);
    }
  }
  __syncthreads();
  // 64 qt rows x 64 bytes: thread t writes 16 bytes of row t / 4.
  const int cc = t >> 2, seg = (t & 3) * 16;
  if (c0 + cc < in && p0 + seg < out)
    *(uint4*)(qt + ((size_t)e * in + c0 + cc) * out + p0 + seg) = *(const uint4*)&tile[cc][seg];
}

__global__ void __launch_bounds__(256) fill_zero_kernel(uint32_t* __restrict__ p, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

__global__ void __launch_bounds__(256) col_scale_kernel(float* __restrict__ scales_t, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) scales_t[i] = fmaxf(scales_t[i] * kInv448, kMinScale);
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
                                                       void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0,
                 "swiglu_quantize_rows_current: I must be a multiple of 8");
  MI355X_REQUIRE(rows >= 0, "swiglu_quantize_rows_current: negative rows");
  if (rows == 0) return MI355X_OK;
  hipLaunchKernelGGL(swiglu_rows_current_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)h, rows, width, limit, q, scales);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_quantize_weights_current_fp8(const void* w, int is_fp32, int experts,
                                                   int out, int in, int interleave, uint8_t* q,
                                                   float* scales, uint8_t* qt, float* scales_t,
                                                   void* stream) {
  MI355X_REQUIRE(experts > 0 && out > 0 && in > 0, "quantize_weights_current: empty weight");
  MI355X_REQUIRE(in % 8 == 0, "quantize_weights_current: in must be a multiple of 8");
  MI355X_REQUIRE(out % 16 == 0, "quantize_weights_current: out must be a multiple of 16");
  hipStream_t s = (hipStream_t)stream;
  const size_t ncol = (size_t)experts * in;
  uint32_t* col_bits = (uint32_t*)scales_t;  // column maxima, then scales in place
  const dim3 amax_grid((out + kAmaxRows - 1) / kAmaxRows, experts);
  const dim3 tile_grid((in + kQTile - 1) / kQTile, (out + kQTile - 1) / kQTile, experts);
  const unsigned lin = (unsigned)((ncol + 255) / 256);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(lin), dim3(256), 0, s, col_bits, ncol);
  if (is_fp32) {
    hipLaunchKernelGGL(weight_amax_kernel<float>, amax_grid, dim3(256), 0, s, (const float*)w,
                       out, in, interleave, scales, col_bits);
    hipLaunchKernelGGL(weight_quantize_kernel<float>, tile_grid, dim3(256), 0, s, (const float*)w,
                       out, in, interleave, scales, col_bits, q, qt);
  } else {
    hipLaunchKernelGGL(weight_amax_kernel<uint16_t>, amax_grid, dim3(256), 0, s,
                       (const uint16_t*)w, out, in, interleave, scales, col_bits);
    hipLaunchKernelGGL(weight_quantize_kernel<uint16_t>, tile_grid, dim3(256), 0, s,
                       (const uint16_t*)w, out, in, interleave, scales, col_bits, q, qt);
  }
  hipLaunchKernelGGL(col_scale_kernel, dim3(lin), dim3(256), 0, s, scales_t, ncol);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}

extern "C" int mi355x_permute_quantize_current_fp8(const void* x, int tokens, int width,
                                                   int top_k, const int32_t* slots, uint8_t* q,
                                                   float* scales, void* stream) {
  MI355X_REQUIRE(width > 0 && width % 8 == 0,
                 "permute_quantize_current: width must be a multiple of 8");
  MI355X_REQUIRE(top_k > 0 && top_k <= 64, "permute_quantize_current: top_k must be in [1, 64]");
  MI355X_REQUIRE(tokens >= 0, "permute_quantize_current: negative tokens");
  if (tokens == 0) return MI355X_OK;
  hipLaunchKernelGGL(permute_rows_current_kernel, dim3((tokens + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x, tokens, width, top_k, slots, q,
                     scales);
  MI355X_LAUNCH_CHECK();
  return MI355X_OK;
}
