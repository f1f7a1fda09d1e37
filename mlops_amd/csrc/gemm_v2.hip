// Grouped block-FP8 GEMM, pipelined form (N a multiple of 256): projection
// (y = x @ W^T), input gradient (dx = dy @ W through the transposed copy) and
// the gate/up-interleaved up projection. See gemm_pipe.h for the tiling.
#include "gemm_pipe.h"

using namespace pipe;

namespace {

constexpr int kMaxExperts = 512;

// Scalar description of one output tile.
struct Tile {
  int e, row0, nvalid, nt;
  int rot;  // K-step rotation: the tile walks K steps rot, rot + 1, ... (mod nk)
  int par;  // which of the two gathered-row tables holds this tile's A rows
};

__device__ __forceinline__ Tile describe(const int* prefix, const int32_t* __restrict__ offsets,
                                         int experts, int n_tiles, int tile, int nk, int n_group,
                                         int rotate) {
  // Every field is wave-uniform; readfirstlane lets the compiler keep them
  // (and everything derived: weight bases, scale addresses) in SGPRs.
  Tile t;
  int mt = tile / n_tiles;
  t.nt = tile % n_tiles;
  t.e = __builtin_amdgcn_readfirstlane(find_expert(prefix, experts, mt));
  if (n_group > 0) {
    // Inside the expert: groups of n_group N tiles (the last may be
    // narrower), each walked over all the expert's row blocks, N fastest.
    // An expert that owns a tile has at least one row block.
    const int blocks = prefix[t.e + 1] - prefix[t.e];
    const int local = tile - prefix[t.e] * n_tiles;
    const int g = local / (blocks * n_group);
    const int gs = min(n_group, n_tiles - g * n_group);
    const int idx = local - g * blocks * n_group;
    mt = __builtin_amdgcn_readfirstlane(prefix[t.e] + idx / gs);
    t.nt = __builtin_amdgcn_readfirstlane(g * n_group + idx % gs);
  }
  t.row0 = __builtin_amdgcn_readfirstlane(offsets[t.e] + (mt - prefix[t.e]) * BM);
  t.nvalid = __builtin_amdgcn_readfirstlane(min(BM, offsets[t.e + 1] - t.row0));
  // Tiles that share an operand panel run at the same time on neighbouring
  // CUs of one XCD; consecutive tiles start one K step apart, over a window
  // of three steps, so that one of them takes a panel step's L2 miss and the
  // others find the line in L2 a step later. The window is kept small: a
  // rotation over all K steps (7t mod nk) took the same time but spread an
  // expert's ~30 concurrent tiles over its whole 5 MB of panels, more than a
  // 4 MB L2, and the up projection read its operands 3.6 times from HBM
  // instead of 1.05 times (2% faster over C3's four launches). Short K
  // (under 8 steps, e.g. the down projection) keeps the full rotation, which
  // measured ~3% faster there, with panels small enough to stay in L2. The
  // grouped order runs unrotated: there the CUs sharing a panel read it
  // together.
  t.rot = rotate ? __builtin_amdgcn_readfirstlane(nk >= 8 ? tile % 3 : (tile * 7) % nk) : 0;
  t.par = 0;
  return t;
}

// Weight row feeding B-tile row `tr` (0..255). Inside each wave's 128
// columns, MFMA column c of block jb is routed to output column c * 8 + jb,
// so a lane's eight accumulator blocks are eight consecutive output columns
// (one 16-byte store per row in the epilogue). Gate/up mode: the wave's
// output columns 2j, 2j+1 hold gate_j, up_j for 64 consecutive j; blocks
// 0-3 carry gates and 4-7 ups of j = jw + 4c + (jb % 4).
__device__ __forceinline__ int weight_row(int tr, int nt, int interleave, int half_n) {
  const int part = tr >> 7, local = tr & 127;  // part = the wave column (wn)
  const int jb = local >> 4, c = local & 15;
  if (!interleave) return nt * BN + part * 128 + c * 8 + jb;
  const int jw = nt * 128 + part * 64;
  const int j = jw + 4 * c + (jb & 3);
  return jb < 4 ? j : half_n + j;
}

typedef short v4s __attribute__((ext_vector_type(4)));

// kRow: row-scaled operands (one descale per activation row, a_scale[rows],
// and one per weight output row, w_scale[E, N]): the K loop accumulates in
// the MFMA itself and the epilogue applies (acc * a_scale) * w_scale once.
// kKM: the weight is read as stored, [E, K, N] (K-major: the input-gradient
// GEMMs on the forward weights, no transposed copy). Its tiles are copied as
// 128 K rows of 256 bytes and the B fragments read with ds_read_b64_tr_b8;
// the MFMA columns are then the tile's columns in order, so the epilogue
// regroups each row's values through LDS into 8-column stores.
// x / d for the divisor d encoded by row_div_magic (s == 0: d = 1): the
// round-down multiply-high method for unsigned division by an invariant
// integer (Granlund and Montgomery, PLDI 1994), with a 33-bit multiplier
// 2^32 + m, exact for every 32-bit x.
__device__ __forceinline__ uint32_t div_rows(uint32_t x, uint32_t m, int s) {
  const uint32_t t = __umulhi(x, m);
  const uint32_t q = (t + ((x - t) >> 1)) >> (s > 0 ? s - 1 : 0);
  return s == 0 ? x : q;  // a select: no branch around the LDS reads it feeds
}

// MFMA block of a K step at which waves 4-7 issue the next step's copies.
constexpr int kLateIssueBlock = 1;

template <bool kAct, bool kAdd, bool kLora, bool kRow = false, bool kKM = false,
          bool kGather = false>
__global__ void __launch_bounds__(kThreads, 2) grouped_gemm_v2_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ a_scale, int rows,
    const uint8_t* __restrict__ w, const float* __restrict__ w_scale, int w_scale_t, int experts,
    int N, int K, const int32_t* __restrict__ offsets, int interleave,
    const uint16_t* __restrict__ addend, uint16_t* __restrict__ out,
    uint8_t* __restrict__ act_q, float* __restrict__ act_scales, float limit,
    const uint16_t* __restrict__ lora_z, const uint16_t* __restrict__ lora_b, int lora_rank,
    int n_group, int rotate, const int32_t* __restrict__ a_rows, int scale_pitch,
    uint32_t div_m, int div_s) {
  __shared__ __align__(1024) uint8_t smem[kStages * STAGE_BYTES];
  __shared__ float act_amax[2][BM];  // per-row amax of each wave column's 64 act columns
  __shared__ int prefix[kMaxExperts + 1];
  __shared__ int tmp[kThreads];
  // Gathered A (kGather): GEMM row r reads a[tok] and its scales
  // a_scale[tok * (K/128) + kb] (token-major), tok = a_rows[r] / d with the
  // divisor d given as (div_m, div_s) (row_div_magic): d = top_k turns the
  // plan's sorted slot order into token rows, d = 1 takes token ids. The
  // activation
  // quantized once per token, each token row read by its k routed rows. A
  // tile's 256 source rows are copied into one of two tables one tile ahead.
  __shared__ int gtok[2][BM];
  tile_prefix(offsets, experts, BM, prefix, tmp);
  const int n_tiles = N / BN;
  const int total = __builtin_amdgcn_readfirstlane(prefix[experts]) * n_tiles;
  const int nk = K / BK;
  const int kbw = K / 128, nbw = N / 128, half_n = N / 2;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 wave grid
  // B fragment of MFMA block jb of this wave's 128 columns. The K-major
  // form takes the lane id through an empty asm at each step, so its 32
  // per-lane fragment addresses are formed where used instead of being
  // hoisted out of the K loop (live across it, they would spill).
  auto bfrag = [&](const uint8_t* tb, int jb, uint32_t step_lane) -> v8i {
    if constexpr (kKM) return frag_kmajor(tb, wn * 128 + jb * 16, (int)step_lane);
    else return frag(tb, wn * 128 + jb * 16 + (lane & 15), lane);
  };

  // Direct loads of one K step of tile t into stage `stage`.
  const int issue_lane = lane;
  auto issue = [&](const Tile& t, int step, int stage) {
    // The fused-SwiGLU form has no registers to keep the per-lane copy
    // offsets across the K loop: the compiler spilled them, and each scratch
    // reload waited on vmcnt, i.e. on the copies in flight. There the lane id
    // passes through an empty asm so the offsets are recomputed at each issue.
    int lane = issue_lane;
    if constexpr (kAct) {
      uint32_t l = (uint32_t)lane;
      asm volatile("" : "+v"(l));
      lane = (int)l;
    }
    const int kb = __builtin_amdgcn_readfirstlane(step + t.rot < nk ? step + t.rot : step + t.rot - nk);
    uint8_t* base = smem + stage * STAGE_BYTES;
    const size_t koff = (size_t)kb * BK;
    const uint8_t* abase = a + koff;
    const uint8_t* bbase = w + (size_t)t.e * N * K + koff;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int r = (wave * A_LOADS + i) * 8 + (lane >> 3);
      int src;
      if constexpr (kGather) src = (int)div_rows((uint32_t)gtok[t.par][r], div_m, div_s);
      else src = min(t.row0 + r, rows - 1);
      const uint32_t off = (uint32_t)src * (uint32_t)K + 16 * ((lane & 7) ^ swz(r));
      dma16(abase, off, base + (wave * A_LOADS + i) * 1024);
    }
    if constexpr (kKM) {
      // K rows kb*128 .. +127 of the expert's [K, N] weight, columns of the
      // tile: a copy is 4 rows x 256 bytes; unit u of row r lands at u ^ kmsw(r).
      const uint8_t* kbase = w + (size_t)t.e * N * K + (size_t)kb * BK * N + (size_t)t.nt * BN;
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) {
        const int r = (wave * B_LOADS + i) * 4 + (lane >> 4);
        const uint32_t off = (uint32_t)r * (uint32_t)N + 16 * ((lane & 15) ^ kmsw(r));
        dma16(kbase, off, base + A_BYTES + (wave * B_LOADS + i) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) {
        const int tr = (wave * B_LOADS + i) * 8 + (lane >> 3);
        const uint32_t off = (uint32_t)weight_row(tr, t.nt, interleave, half_n) * (uint32_t)K +
                             16 * ((lane & 7) ^ swz(tr));
        dma16(bbase, off, base + A_BYTES + (wave * B_LOADS + i) * 1024);
      }
    }
    if constexpr (kRow) return;  // no per-step scales
    // The step's scales travel in the stage with its operands (an ordinary
    // load here would make the compiler wait on it, and in-order completion
    // would make that wait cover this step's operand copies too), in as few
    // copies as their layout allows: the 256 row scales by waves 0-3, 64
    // rows each, and the two weight block scales of each wave column (its
    // low and high 128 columns) by waves 4-5.
    if (wave < 4) {
      // Gathered: token-major scales [tokens][K/128], a token's K steps on
      // one line; else K-block-major [K/128][rows].
      const float* sbase = kGather ? a_scale + kb : a_scale + (size_t)kb * rows;
      uint32_t off;
      if constexpr (kGather) off = 4u * div_rows((uint32_t)gtok[t.par][wave * 64 + lane], div_m, div_s) * (uint32_t)kbw;
      else off = 4u * (uint32_t)min(t.row0 + wave * 64 + lane, rows - 1);
      dma4(sbase, off, base + A_BYTES + B_BYTES + wave * 256);
    } else if (wave < 6 && lane < 2) {
      const int c = wave - 4;  // wave column
      const int nb = lane == 0 ? (interleave ? t.nt : 2 * t.nt + c)
                               : (interleave ? half_n / 128 + t.nt : 2 * t.nt + c);
      const uint32_t idx = w_scale_t ? (uint32_t)((t.e * kbw + kb) * nbw + nb)
                                     : (uint32_t)((t.e * nbw + nb) * kbw + kb);
      dma4(w_scale, 4u * idx, base + A_BYTES + B_BYTES + SA_BYTES + c * 8);
    }
  };

  // XCD-affine order: workgroup b runs on XCD b % 8, and XCD x takes the
  // x-th eighth of the expert-major tile list (every tile costs the same K
  // steps), so the N tiles of one row block share its activation rows, and
  // the row blocks of one expert share its weight panel, in one XCD's L2.
  // The G/8 workgroups of an XCD take its range round-robin. Needs a grid
  // that is a multiple of 8; otherwise plain order.
  const bool affine = (gridDim.x & 7) == 0;
  const int xcd = blockIdx.x & 7, cu = blockIdx.x >> 3, per_xcd = gridDim.x >> 3;
  const int first = affine ? (int)((long long)total * xcd / 8) : 0;
  const int last = affine ? (int)((long long)total * (xcd + 1) / 8) : total;
  auto tile_at = [&](int r) -> int {
    if (!affine) return tile_of(r, blockIdx.x, gridDim.x);
    const int t = first + r * per_xcd + cu;
    return t < last ? t : total;
  };
  int round = 0;
  int tile = tile_at(0);
  if (tile >= total) return;
  Tile ct = describe(prefix, offsets, experts, n_tiles, tile, nk, n_group, rotate);
  // Gathered A: the tile's 256 source rows (row indices clamped to the last
  // row, as the plain copies clamp) into table `par`, by the first four waves'
  // direct loads; they land before the next wait_and_sync<0> returns.
  auto load_rows = [&](const Tile& t, int par) {
    if (kGather && wave < 4)
      dma4(a_rows, 4u * (uint32_t)min(t.row0 + wave * 64 + lane, rows - 1),
           (const uint8_t*)&gtok[par][wave * 64]);
  };
  if constexpr (kGather) {
    load_rows(ct, 0);
    wait_and_sync<0>();
  }
  issue(ct, 0, 0);
  int stage = 0;
  for (;;) {
    const int next_tile = tile_at(round + 1);
    v4f acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kLora) {
      // The accumulators start from the rank-r product z[row] . b[e][col]
      // (bf16 MFMA, fp32 sums, 16 of the rank at a time): the low-rank term
      // of out = A W^T + z B^T joins before the block products, with no
      // [rows, N] addend in memory. A lane's z fragment is 4 consecutive
      // rank entries of its A row (16x16x16 operand layout), its b fragment
      // 4 of the weight row feeding its B column, the same rows the
      // operand copies use; the result lands in the accumulator layout of
      // the fp8 MFMA.
      const int zl = lane & 15, kq = 4 * (lane >> 4);
      for (int kc = 0; kc < lora_rank; kc += 16) {
        v4s zf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = min(ct.row0 + wm * 64 + i * 16 + zl, rows - 1);
          zf[i] = *(const v4s*)(lora_z + (size_t)row * lora_rank + kc + kq);
        }
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
          const int wrow = weight_row(wn * 128 + jb * 16 + zl, ct.nt, interleave, half_n);
          const v4s bf = *(const v4s*)(lora_b + ((size_t)ct.e * N + wrow) * lora_rank + kc + kq);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[i][jb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(zf[i], bf, acc[i][jb], 0, 0, 0);
        }
      }
      if constexpr (kRow) {
        // The epilogue multiplies the whole accumulator by the row and column
        // descales: the rank term enters divided by them, so it comes out as
        // itself (a few fp32 roundings). Block jb of a lane is output column
        // zl * 8 + jb of the wave's 128, as in the epilogue.
        const float* wsb = w_scale + (size_t)ct.e * N + ct.nt * BN + wn * 128 + zl * 8;
        const float4 w0 = *(const float4*)wsb, w1 = *(const float4*)(wsb + 4);
        const float iw[8] = {1.0f / w0.x, 1.0f / w0.y, 1.0f / w0.z, 1.0f / w0.w,
                             1.0f / w1.x, 1.0f / w1.y, 1.0f / w1.z, 1.0f / w1.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = min(ct.row0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r, rows - 1);
            const float ixs = 1.0f / a_scale[row];
#pragma unroll
            for (int jb = 0; jb < 8; ++jb) acc[i][jb][r] = (acc[i][jb][r] * ixs) * iw[jb];
          }
      }
    }

    for (int kb = 0; kb < nk; ++kb) {
      wait_and_sync<0>();  // two stages: the only loads in flight are this step's
      if (kGather && kb == 0 && next_tile < total) {
        // The next tile's source rows, into the other table (its last reader,
        // the tile before this one, finished before the barrier above). With
        // a single K step they are needed right away.
        load_rows(describe(prefix, offsets, experts, n_tiles, next_tile, nk, n_group, rotate),
                  (round + 1) & 1);
        if (nk == 1) wait_and_sync<0>();
      }
      // Next step's operands (the next tile's first step at the last step:
      // its loads then run under this tile's epilogue). A wave is held at
      // each direct load until the address unit takes it, and waves w and
      // w + 4 share a SIMD: waves 4-7 issue theirs after their first MFMA
      // block instead, so that while one wave of a SIMD is held the other
      // has MFMAs to issue. (A later issue point needs registers the step
      // does not have: the compiler spills.)
      const bool late = wave >= 4 && kb + 1 < nk;
      if (late) {
        // issued in the K step below, at MFMA block kLateIssueBlock
      } else if (kb + 1 < nk) {
        issue(ct, kb + 1, stage ^ 1);
      } else if (next_tile < total) {
        Tile nt = describe(prefix, offsets, experts, n_tiles, next_tile, nk, n_group, rotate);
        if constexpr (kGather) nt.par = (round + 1) & 1;
        issue(nt, 0, stage ^ 1);
      }
      const uint8_t* base = smem + stage * STAGE_BYTES;
      const uint8_t* ta = base;
      const uint8_t* tb = base + A_BYTES;
      if constexpr (kRow) {
        uint32_t klane = lane;
        if constexpr (kKM) asm volatile("" : "+v"(klane));
        v8i bcur = bfrag(tb, 0, klane);
        v8i af[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = frag(ta, wm * 64 + i * 16 + (lane & 15), lane);
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
          if (late && jb == kLateIssueBlock) {
            __builtin_amdgcn_sched_barrier(0);
            issue(ct, kb + 1, stage ^ 1);
            __builtin_amdgcn_sched_barrier(0);
          }
          v8i bnext = bcur;
          if (jb < 7) bnext = bfrag(tb, jb + 1, klane);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i][jb] = mfma_acc(af[i], bcur, acc[i][jb]);
          bcur = bnext;
        }
        stage ^= 1;
        continue;
      }
      const float* sa = (const float*)(base + A_BYTES + B_BYTES);
      const float2 sbw = *(const float2*)(base + A_BYTES + B_BYTES + SA_BYTES + wn * 8);
      const float sb_lo = sbw.x, sb_hi = sbw.y;
      // One B block at a time against the four A blocks (register budget:
      // two waves share a SIMD, 256 registers each), read one block ahead.
      // Reads in use order (first B block, A blocks, then the scales), so
      // the first MFMA waits for two of them rather than for all.
      uint32_t klane = lane;
      if constexpr (kKM) asm volatile("" : "+v"(klane));
      v8i bcur = bfrag(tb, 0, klane);
      v8i af[4];
      float s4[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = frag(ta, wm * 64 + i * 16 + (lane & 15), lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float4 v = *(const float4*)&sa[wm * 64 + i * 16 + 4 * (lane >> 4)];
        s4[i][0] = v.x; s4[i][1] = v.y; s4[i][2] = v.z; s4[i][3] = v.w;
      }
      float sc[4][4];
#pragma unroll
      for (int jb = 0; jb < 8; ++jb) {
        if (late && jb == kLateIssueBlock) {
          __builtin_amdgcn_sched_barrier(0);
          issue(ct, kb + 1, stage ^ 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (jb == 0 || jb == 4) {
          const float sb = jb < 4 ? sb_lo : sb_hi;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[i][r] = s4[i][r] * sb;
        }
        v8i bnext = bcur;
        if (jb < 7) bnext = bfrag(tb, jb + 1, klane);
        v4f p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = mfma(af[i], bcur);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][jb][r] = fmaf(p[i][r], sc[i][r], acc[i][jb][r]);
        bcur = bnext;
      }
      stage ^= 1;
    }

    // ---- epilogue straight from registers: lane (row, 8 consecutive
    // columns) -> one 16-byte store per row, rounding to bf16 once. Wave
    // base pointer + 32-bit per-lane offsets.
    uint16_t* obase = out + (size_t)(ct.row0 + wm * 64) * N + ct.nt * BN + wn * 128;
    // kAdd: a bf16 addend is given (a separate instantiation, so the plain
    // kernel carries none of its registers).
    const uint16_t* cbase = !kAdd ? nullptr
        : addend + (size_t)(ct.row0 + wm * 64) * N + ct.nt * BN + wn * 128;
    // The lane id passes through an empty asm here, so the per-row store
    // addresses are computed where they are used. Hoisted above the K loop
    // (they depend only on the tile and the lane) they would be live across
    // it and spill, and every store would wait on a scratch reload.
    uint32_t elane = lane;
    asm volatile("" : "+v"(elane));
    const uint32_t lane_col = (elane & 15) * 8;
    if constexpr (kKM) {
      // The lane holds column jb*16 + lane%16 of each block: the rows go
      // through this wave's 8 KB of the stage the last step read (32 rows
      // at a time, natural column order), and come back as 8 consecutive
      // columns per lane for one 16-byte store per row, as below.
      static_assert(!kAct && !kAdd && !kLora && !kRow, "K-major weights: plain form only");
      lds_sync();  // every wave is done with the last step's fragments
      uint16_t* st = (uint16_t*)(smem + (stage ^ 1) * STAGE_BYTES) + wave * (32 * 128);
      const uint32_t l16 = elane & 15, lg = elane >> 4;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int jb = 0; jb < 8; ++jb)
              st[(ii * 16 + 4 * lg + r) * 128 + jb * 16 + l16] =
                  f32_to_bf16(acc[half * 2 + ii][jb][r]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t lrow = ii * 16 + 4 * lg + r;
            const uint4 o = *(const uint4*)&st[lrow * 128 + lane_col];
            const uint32_t orow = half * 32 + lrow;  // row within the wave's 64
            if (wm * 64 + (int)orow < ct.nvalid)
              store_stream(obase + orow * (uint32_t)N + lane_col, o);
          }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    } else {
    // kRow: the lane's 8 output columns' weight descales.
    float wsc[8];
    if constexpr (kRow) {
      const float* wsb = w_scale + (size_t)ct.e * N + ct.nt * BN + wn * 128 + lane_col;
      const float4 w0 = *(const float4*)wsb, w1 = *(const float4*)(wsb + 4);
      wsc[0] = w0.x; wsc[1] = w0.y; wsc[2] = w0.z; wsc[3] = w0.w;
      wsc[4] = w1.x; wsc[5] = w1.y; wsc[6] = w1.z; wsc[7] = w1.w;
    }
    // SwiGLU fused into the up projection (gate/up mode with act_q): the
    // activation of the stored bf16 gate/up pairs, quantized 1x128 as
    // swiglu_quantize_kernel does. A lane holds 4 of a row's 64 act columns
    // in this wave; the 128-column group spans both wave columns (wn), whose
    // row maxima meet in LDS.
    constexpr bool act_out = kAct;  // act_q != nullptr
    // Row groups of the wave (kParts of them), each: store h and keep the
    // activations, exchange row maxima, quantize and store act. With the
    // activations one 16-row block at a time (four exchanges) the epilogue
    // fits the registers; two blocks at a time spilled inside the K loop.
    constexpr int kParts = act_out ? 4 : 2, kPer = 4 / kParts;
#pragma unroll
    for (int half = 0; half < kParts; ++half) {
      float act[kPer][4][4];
      // The addend's 8 rows of this half, loaded before its first store:
      // loads and stores share one completion counter, so a load issued
      // after a store would wait for that store too.
      uint4 cadd[kPer][4];
      if (kAdd) {
#pragma unroll
        for (int ii = 0; ii < kPer; ++ii)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int lrow = (half * kPer + ii) * 16 + 4 * (elane >> 4) + r;
            cadd[ii][r] = make_uint4(0, 0, 0, 0);
            if (wm * 64 + lrow < ct.nvalid)
              cadd[ii][r] = *(const uint4*)(cbase + (uint32_t)lrow * (uint32_t)N + lane_col);
          }
      }
#pragma unroll
      for (int ii = 0; ii < kPer; ++ii) {
        const int i = half * kPer + ii;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lrow = i * 16 + 4 * (elane >> 4) + r;  // row within the wave's 64
          float v[8];
          if (interleave) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              v[2 * m] = acc[i][m][r];
              v[2 * m + 1] = acc[i][4 + m][r];
            }
          } else {
#pragma unroll
            for (int m = 0; m < 8; ++m) v[m] = acc[i][m][r];
          }
          if (wm * 64 + lrow < ct.nvalid) {
            const uint32_t off = (uint32_t)lrow * (uint32_t)N + lane_col;
            if constexpr (kRow) {
              float xs;
              if constexpr (kGather) xs = a_scale[div_rows((uint32_t)gtok[ct.par][wm * 64 + lrow], div_m, div_s)];
              else xs = a_scale[ct.row0 + wm * 64 + lrow];
#pragma unroll
              for (int m = 0; m < 8; ++m) v[m] = (v[m] * xs) * wsc[m];
            }
            if (kAdd) {
              const uint4 c = cadd[ii][r];
              uint32_t w4[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                v[2 * m] += bf16_to_f32(w4[m] & 0xffff);
                v[2 * m + 1] += bf16_to_f32(w4[m] >> 16);
              }
            }
            uint4 o;
            o.x = pack_bf16x2(v[0], v[1]);
            o.y = pack_bf16x2(v[2], v[3]);
            o.z = pack_bf16x2(v[4], v[5]);
            o.w = pack_bf16x2(v[6], v[7]);
            store_stream(obase + off, o);
            if (act_out) {
              const uint32_t w4[4] = {o.x, o.y, o.z, o.w};
              float pmax = 0.0f;
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                float g = bf16_to_f32(w4[m] & 0xffff), u = bf16_to_f32(w4[m] >> 16);
                clamp_gate_up(g, u, limit);
                act[ii][r][m] = silu_f(g) * u;
                pmax = fmaxf(pmax, fabsf(act[ii][r][m]));
              }
              pmax = group_amax<16>(pmax);  // the 16 lanes of this row: 64 columns
              if ((elane & 15) == 0) act_amax[wn][wm * 64 + lrow] = pmax;
            }
          }
        }
      }
      if (act_out) {
        lds_sync();
        const int half_w = N / 2;
#pragma unroll
        for (int ii = 0; ii < kPer; ++ii) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int trow = wm * 64 + (half * kPer + ii) * 16 + 4 * (elane >> 4) + r;
            if (trow < ct.nvalid) {
              const float amax = fmaxf(act_amax[0][trow], act_amax[1][trow]);
              const float sc = fmaxf(amax * kInv448, kMinScale);
              const uint32_t qv =
                  f32x4_to_e4m3(quant_div(act[ii][r][0], sc), quant_div(act[ii][r][1], sc),
                                quant_div(act[ii][r][2], sc), quant_div(act[ii][r][3], sc));
              const size_t row = (size_t)(ct.row0 + trow);
              *(uint32_t*)(act_q + row * half_w + ct.nt * 128 + wn * 64 + (elane & 15) * 4) = qv;
              if (wn == 0 && (elane & 15) == 0) act_scales[(size_t)ct.nt * rows + row] = sc;
            }
          }
        }
      }
    }
    }  // not kKM
    if (next_tile >= total) break;
    ++round;
    tile = next_tile;
    ct = describe(prefix, offsets, experts, n_tiles, tile, nk, n_group, rotate);
    if constexpr (kGather) ct.par = round & 1;
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

// Tile order by the size of one expert's weight (N x K bytes). Up to a few
// L2s' worth, tiles go row-block-major with the K rotation: an XCD's CUs
// sweep one row block's N tiles, and the whole weight stays cached across
// row blocks. Beyond that, each row block would stream the weight again
// from HBM, so tiles go in groups of 8 N tiles x all the expert's row
// blocks, unrotated, and the CUs that share a weight panel read it
// together. Measured on MI355X: Mixtral's four GEMMs (58-117 MB per
// expert) +6-14%, DeepSeek-shard up/dgrad-up (29 MB) +5-7%; the 3-15 MB
// weights of the other shapes lose 1-7% in that order.
namespace {
struct Order {
  int n_group, rotate;
};
Order tile_order(int n, int k) {
  if ((size_t)n * (size_t)k >= ((size_t)24 << 20)) return {8, 0};
  return {0, 1};
}
}  // namespace

// (m, s) for div_rows: s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1
// for d >= 2; (0, 0) for d = 1.
struct RowDiv {
  uint32_t m;
  int s;
};
RowDiv row_div_magic(int d) {
  if (d <= 1) return {0u, 0};
  int s = 0;
  while ((1 << s) < d) ++s;
  const uint64_t m = (((uint64_t)1 << 32) * (uint64_t)((1 << s) - d)) / (uint64_t)d + 1;
  return {(uint32_t)m, s};
}

// Launches the pipelined kernel; returns 1 if the shape is not its form
// (N % 256 != 0), in which case the caller uses the general kernel.
int mi355x_gemm_v2_launch(const uint8_t* a, const float* a_scale, int rows, const uint8_t* w,
                          const float* w_scale, int w_scale_t, int experts, int n, int k,
                          const int32_t* offsets, int interleave, const void* addend, void* out,
                          uint8_t* act_q, float* act_scales, float limit, const void* lora_z,
                          const void* lora_b, int lora_rank, void* stream,
                          const int32_t* a_rows, int a_total, int a_rows_div) {
  if (n % BN != 0 || experts > kMaxExperts || (interleave && (n / 2) % 128 != 0)) return 1;
  const RowDiv div = row_div_magic(a_rows_div);
  const int upper = ((rows + BM - 1) / BM + experts) * (n / BN);
  const int grid = upper < cu_count() ? upper : cu_count();
  const Order order = tile_order(n, k);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a, a_scale,
                       rows, w, w_scale, w_scale_t, experts, n, k, offsets, interleave,
                       (const uint16_t*)addend, (uint16_t*)out, act_q, act_scales, limit,
                       (const uint16_t*)lora_z, (const uint16_t*)lora_b, lora_rank,
                       order.n_group, order.rotate, a_rows, a_rows != nullptr ? a_total : rows, div.m, div.s);
  };
  if (a_rows != nullptr) {
    if (lora_z != nullptr || act_q != nullptr || addend != nullptr) return 1;
    launch(grouped_gemm_v2_kernel<false, false, false, false, false, true>);
  } else if (lora_z != nullptr) {
    if (act_q != nullptr || addend != nullptr) return 1;  // not a form of this kernel
    launch(grouped_gemm_v2_kernel<false, false, true>);
  } else if (act_q != nullptr) {
    addend != nullptr ? launch(grouped_gemm_v2_kernel<true, true, false>)
                      : launch(grouped_gemm_v2_kernel<true, false, false>);
  } else {
    addend != nullptr ? launch(grouped_gemm_v2_kernel<false, true, false>)
                      : launch(grouped_gemm_v2_kernel<false, false, false>);
  }
  MI355X_LAUNCH_CHECK();
  return 0;
}

// K-major weight (see kKM): w [E, K, N] e4m3 with its own block scales
// [E, K/128, N/128]; returns 1 if the shape is not this kernel's (N % 256).
int mi355x_gemm_v2_kmajor_launch(const uint8_t* a, const float* a_scale, int rows,
                                 const uint8_t* w, const float* w_scale, int experts, int n, int k,
                                 const int32_t* offsets, void* out, void* stream,
                                 const int32_t* a_rows, int a_total, int a_rows_div) {
  if (n % BN != 0 || experts > kMaxExperts) return 1;
  const RowDiv div = row_div_magic(a_rows_div);
  const int upper = ((rows + BM - 1) / BM + experts) * (n / BN);
  const int grid = upper < cu_count() ? upper : cu_count();
  const Order order = tile_order(n, k);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a, a_scale,
                       rows, w, w_scale, 1, experts, n, k, offsets, 0, (const uint16_t*)nullptr,
                       (uint16_t*)out, (uint8_t*)nullptr, (float*)nullptr, 0.0f,
                       (const uint16_t*)nullptr, (const uint16_t*)nullptr, 0, order.n_group,
                       order.rotate, a_rows, a_rows != nullptr ? a_total : rows, div.m, div.s);
  };
  if (a_rows != nullptr) launch(grouped_gemm_v2_kernel<false, false, false, false, true, true>);
  else launch(grouped_gemm_v2_kernel<false, false, false, false, true>);
  MI355X_LAUNCH_CHECK();
  return 0;
}

// Row-scaled form (see kRow): a_scale [rows], w_scale [E, N]; returns 1 if
// the shape is not this kernel's (N % 256 != 0).
int mi355x_gemm_v2_rowwise_launch(const uint8_t* a, const float* a_scale, int rows,
                                  const uint8_t* w, const float* w_scale, int experts, int n,
                                  int k, const int32_t* offsets, const void* lora_z,
                                  const void* lora_b, int lora_rank, void* out, void* stream,
                                  const int32_t* a_rows, int a_total, int a_rows_div) {
  if (n % BN != 0 || experts > kMaxExperts) return 1;
  const RowDiv div = row_div_magic(a_rows_div);
  const int upper = ((rows + BM - 1) / BM + experts) * (n / BN);
  const int grid = upper < cu_count() ? upper : cu_count();
  const Order order = tile_order(n, k);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a, a_scale,
                       rows, w, w_scale, 0, experts, n, k, offsets, 0, (const uint16_t*)nullptr,
                       (uint16_t*)out, (uint8_t*)nullptr, (float*)nullptr, 0.0f,
                       (const uint16_t*)lora_z, (const uint16_t*)lora_b, lora_rank,
                       order.n_group, order.rotate, a_rows, a_rows != nullptr ? a_total : rows, div.m, div.s);
  };
  if (a_rows != nullptr) {
    if (lora_z != nullptr) return 1;  // not a form of this kernel
    launch(grouped_gemm_v2_kernel<false, false, false, true, false, true>);
  } else if (lora_z != nullptr) launch(grouped_gemm_v2_kernel<false, false, true, true>);
  else launch(grouped_gemm_v2_kernel<false, false, false, true>);
  MI355X_LAUNCH_CHECK();
  return 0;
}
