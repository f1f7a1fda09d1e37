// Pipelined block-FP8 MFMA main loop for gfx950, shared by the grouped GEMMs.
//
// Workgroup tile 256 (M) x 256 (N) x 128 (K), 8 waves (two per SIMD) in a
// 4 x 2 grid, wave tile 64 x 128 (4 x 8 blocks of
// v_mfma_f32_16x16x128_f8f6f4). Operands are copied global -> LDS by the
// CDNA4 direct loads (global_load_lds_dwordx4: no staging registers, no LDS
// store instructions) into two stages, one s_barrier per K step.
//
// Why 256 x 256: the L2 -> LDS direct-load path sustains ~54 B/clk/CU on
// MI355X (measured); a K step of this tile moves 64 KB for 16.8 MFLOP
// (256 flop/B), so the copy takes ~60% of the MFMA time and hides under it,
// where a 128 x 256 tile (171 flop/B) would make the GEMM copy-bound.
//
// LDS rows are 128 bytes, unpadded; the 16-byte unit c of row r is stored at
// unit c ^ (r & 7). A fragment lane (row l % 16, group g = l / 16) takes the
// units g and g + 4 of its row: A and B lanes agree on that K assignment, so
// the MFMA sum is unchanged, and a wave's 16 rows x 4 units per read then
// hit every bank once (measured on MI355X: full LDS read bandwidth, against
// ~63% for adjacent unit pairs under any row swizzle).
// A direct load writes 64 lanes x 16 B = 8 rows; lane L writes unit L % 8 of
// row L / 8 and so loads the logical unit (L % 8) ^ swizzle(row).
#pragma once

#include "common.h"

namespace pipe {

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 2;
constexpr int A_BYTES = BM * BK;          // 32 KB
constexpr int B_BYTES = BN * BK;          // 32 KB
constexpr int SA_BYTES = BM * 4;          // row scales of A
constexpr int SB_BYTES = BN * 4;          // column scales of B (weight-gradient form)
constexpr int STAGE_BYTES = A_BYTES + B_BYTES + SA_BYTES + SB_BYTES;
constexpr int A_LOADS = A_BYTES / 1024 / kWaves;  // direct loads per wave per stage: 4
constexpr int B_LOADS = B_BYTES / 1024 / kWaves;  // 4

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ int swz(int row) { return row & 7; }

// The direct loads are issued as inline assembly, invisible to the
// compiler's wait-count bookkeeping: it would otherwise wait for every
// in-flight load before any LDS read it cannot prove disjoint. The kernels
// count their own loads and wait with wait_and_sync<N>.
// LDS byte address of a (wave-uniform) LDS pointer, as a scalar for M0.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr_t)p);
}
// Source address = wave-uniform 64-bit base (SGPRs) + per-lane 32-bit byte
// offset (one VGPR), the saddr form of the global load.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, const uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr(lds)), "v"(off), "s"(base) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, const uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :: "s"(lds_addr(lds)), "v"(off), "s"(base) : "memory", "m0");
}

// Wait until at most N direct loads of this wave are in flight, then barrier.
template <int N>
__device__ __forceinline__ void wait_and_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt[3:0], expcnt[6:4]=7, lgkmcnt[11:8]=15, vmcnt[5:4] in [15:14]
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Barrier that waits for this wave's LDS operations only (not for its
// in-flight global loads and stores).
__device__ __forceinline__ void lds_sync() {
  // vmcnt = 63 (no wait), expcnt = 7, lgkmcnt = 0
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void sync_all() {
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 32 fp8 K-values of one fragment row from a swizzled stage tile.
__device__ __forceinline__ v8i frag(const uint8_t* tile, int row, int lane) {
  const int g = lane >> 4;  // units g and g + 4
  const int s = swz(row);
  const uint8_t* base = tile + row * 128;
  uint4 x = *(const uint4*)(base + 16 * (g ^ s));
  uint4 y = *(const uint4*)(base + 16 * ((g + 4) ^ s));
  v8i r;
  r[0] = x.x; r[1] = x.y; r[2] = x.z; r[3] = x.w;
  r[4] = y.x; r[5] = y.y; r[6] = y.z; r[7] = y.w;
  return r;
}

// Position of 16-byte unit u in row r of a K-major stage tile: u ^ kmsw(r).
// A fragment read takes rows r .. r+7 (r % 8 == 0) in each 16-lane group and
// rows 16 apart across the four groups of a wave: the low bits spread a
// group's rows over 8 positions, and bit 3 (row / 16 odd) moves the odd
// groups to the other 8, so a 64-lane read meets each bank twice.
__device__ __forceinline__ int kmsw(int r) { return (r & 15) ^ (((r >> 4) & 1) << 3); }

// The same fragment (32 fp8 K-values of one B column) from a K-major stage
// tile: 128 K rows of 256 bytes (one byte per column), 16-byte unit u of row
// r stored at u ^ kmsw(r). ds_read_b64_tr_b8 gives lane j of each 16-lane
// group byte (j % 8) of the 8 bytes addressed by lane 2b + j / 8, as its
// byte b; so with lane i addressing K row kbase + i / 2 at column
// col0 + 8 (i % 2), lane j receives column col0 + j at K rows kbase .. +7.
// Four such reads give the K rows of frag(): 16g .. 16g+15 and
// 64+16g .. 64+16g+15 (g = lane / 16).
typedef int v2i_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v8i frag_kmajor(const uint8_t* tile, int col0, int lane) {
  const int g = lane >> 4, j = lane & 15;
  const int unit = col0 >> 4;
  v8i r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int row = (p >> 1) * 64 + 16 * g + (p & 1) * 8 + (j >> 1);
    const uint8_t* at = tile + row * 256 + 16 * (unit ^ kmsw(row)) + 8 * (j & 1);
    const v2i_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i_t*)(lds_ptr_t)at);
    r[2 * p] = v[0];
    r[2 * p + 1] = v[1];
  }
  return r;
}

__device__ __forceinline__ v4f mfma(v8i a, v8i b) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// The same MFMA accumulating into c (row-scaled operands: no per-block fold).
__device__ __forceinline__ v4f mfma_acc(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Exclusive prefix of ceil(rows_e / tile) over experts -> prefix[0..E].
__device__ inline void tile_prefix(const int32_t* __restrict__ offsets, int experts, int tile,
                                   int* prefix, int* tmp) {
  const int t = threadIdx.x;
  const int per = (experts + kThreads - 1) / kThreads;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    int e = t * per + i;
    if (e < experts) local += (offsets[e + 1] - offsets[e] + tile - 1) / tile;
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
      run += (offsets[e + 1] - offsets[e] + tile - 1) / tile;
    }
  }
  if (t == kThreads - 1) prefix[experts] = tmp[t];
  __syncthreads();
}

__device__ __forceinline__ int find_expert(const int* prefix, int experts, int tile) {
  int lo = 0, hi = experts - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Persistent tile order: in each round of G tiles, XCD x (= block % 8) takes
// the G/8 consecutive tiles starting at x * G/8, so the 32 CUs of one XCD
// share A rows across N tiles and weights across M tiles in their L2.
// Round-robin tile assignment. Grouping consecutive tiles onto one XCD (block
// b runs on XCD b % 8) raised the L2 hit rate from ~10% to ~64% but measured
// 5-20% slower on the MoE and dense shapes, so tiles go out in plain order.
__device__ __forceinline__ int tile_of(int round, int block, int grid) {
  return round * grid + block;
}

}  // namespace pipe
