// 256x256 FP8 tile engine fed by direct global->LDS DMA (gfx950
// global_load_lds_dwordx4), shared by the dense and the grouped expert GEMMs.
//
// C[m, n] = sum_kb ( A_kb[m, :] . B_kb[n, :] ) * as[m, kb] * ws[n / 128, kb]
//
// Workgroup: 8 waves (512 threads), tile 256 (A rows) x 256 (B rows) x 128.
// Wave w multiplies A rows 64*(w%4) .. +63 against B rows 128*(w/4) .. +127,
// so its B rows sit in one 128-row weight-scale block and the weight scale
// of a k-block is one number per wave.
//
// LDS: two stages, each A tile (32 KB) then B tile (32 KB), 128-byte rows of
// 16-byte chunks; chunk c of row r sits at slot c ^ swizzle(r) with
// swizzle(r) = (r & 7) ^ ((r >> 3) & 1), which puts the 16 rows x 16 bytes read by
// one quarter-wave of ds_read_b128 on 16 distinct 16-byte bank groups of the
// 256-byte-wide LDS.  Each stage is its own __shared__ array and is selected
// at compile time, so the compiler can tell that reads of one stage never
// alias the DMA writes into the other one and does not wait for them.
//
// DMA: one global_load_lds_dwordx4 moves 64 lanes x 16 bytes into 1 KB of
// LDS at M0 + 16 * lane, i.e. 8 consecutive 128-byte tile rows.  The lane
// that lands in slot (lane & 7) of row r therefore fetches logical chunk
// (lane & 7) ^ swizzle(r) of that row.  Each wave moves 8 KB (one quarter of
// A for waves 0-3, of B for waves 4-7) per k-block, one piece per n-tile of
// the multiply, so the copy engine runs while the MFMAs of the current stage
// are issued; waves 0-3 also copy the 256 activation scales of the k-block.
//
// MFMA operands are swapped (weight fragment first), so lane l of a 16x16
// product holds output row m = l % 16 and the four consecutive output columns
// n = 4 * (l / 16) + e: the per-row activation scale is one value per lane
// and the epilogue writes 4 adjacent columns per lane.
#pragma once

#include "common.h"

namespace akas {
namespace dma {

constexpr int BM = 256, BN = 256, THREADS = 512;
constexpr int STAGE = (BM + BN) * 128;

typedef __attribute__((address_space(3))) void lds_void;

static __shared__ __attribute__((aligned(1024))) uint8_t stage0[STAGE];
static __shared__ __attribute__((aligned(1024))) uint8_t stage1[STAGE];
static __shared__ __attribute__((aligned(16))) float scales0[BM];
static __shared__ __attribute__((aligned(16))) float scales1[BM];
// Weight scales of a tile's two 128-row B blocks, one per k-block of the
// workgroup's k range (at most MAX_KB k-blocks).
constexpr int MAX_KB = 128;
static __shared__ __attribute__((aligned(16))) float wtab[2][MAX_KB];

template <int S> AKAS_DEV uint8_t* stage_base() { return S ? stage1 : stage0; }
template <int S> AKAS_DEV float* stage_scales() { return S ? scales1 : scales0; }

AKAS_DEV int swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }
AKAS_DEV int tile_off(int row, int chunk) { return row * 128 + ((chunk ^ swizzle(row)) << 4); }

AKAS_DEV v8i fragment(const uint8_t* tile, int row0, int lane) {
  const int row = row0 + (lane & 15), g = lane >> 4;
  const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + tile_off(row, 2 * g));
  const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + tile_off(row, 2 * g + 1));
  v8i f;
  f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
  f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
  return f;
}

// Tile row (0..255) of this lane in DMA piece i of a wave's quarter tile.
AKAS_DEV int piece_row(int wave, int i, int lane) { return ((wave & 3) * 8 + i) * 8 + (lane >> 3); }
// Byte offset within a source row of the chunk this lane fetches for tile row `row`.
AKAS_DEV int piece_chunk(int row, int lane) { return ((lane & 7) ^ swizzle(row)) << 4; }

// Per-wave copy plans.  ptr(i, ko) is the address of the 16 bytes this lane
// copies for piece i of the k-block at byte offset ko; rows past an
// operand's end are clamped to a valid row (their products are never stored).
//
// AffinePlan: the wave's source rows are row0 + 8*i (+ lane/8 folded into
// row0), clamped to lim -- contiguous operands.  The tile row of piece i is
// 8*i below that of piece 0, whose bit 3 is clear, so its swizzle differs
// from piece 0's in bit 0 exactly when i is odd: the chunk of piece i is
// chunk ^ ((i & 1) << 4).
struct AffinePlan {
  const uint8_t* src;   // A codes for waves 0-3, B codes for waves 4-7
  uint32_t row0;        // this lane's source row for piece 0
  uint32_t lim;         // last valid source row
  uint32_t ld;          // source row stride in bytes
  uint32_t chunk;       // byte offset of this lane's chunk within a row (piece 0)
  int blk0;             // first 1 KB LDS block of this wave within a stage
  const float* as;      // activation scales (waves 0-3)
  uint32_t soff;        // this lane's activation-scale offset (row * KB)
  bool scales;          // wave copies activation scales
  // Every row of the wave's quarter is past the operand: no copies.  Only
  // honoured by a wave that multiplies nothing (run with live false); the
  // stage then keeps stale bytes in that quarter, so a wave may set it only
  // when those rows feed no stored output.
  bool skip;
  AKAS_DEV const uint8_t* ptr(int i, uint32_t ko) const {
    return src + (min(row0 + 8u * i, lim) * ld + (chunk ^ ((i & 1) << 4)) + ko);
  }
};

// GatherPlan: one arbitrary source offset per piece (rows gathered through
// a route table, or weight rows of two banks); piece i reads from
// src + alt_delta instead of src when bit i of the wave-uniform alt_mask is
// set.  (The bank is chosen by adding an integer, not by selecting between
// two pointer fields, which would keep the plan in scratch memory.)
struct GatherPlan {
  const uint8_t* src;
  int64_t alt_delta;
  uint32_t alt_mask;
  uint32_t off[8];
  int blk0;
  const float* as;
  uint32_t soff;
  bool scales;
  bool skip;  // as in AffinePlan
  AKAS_DEV const uint8_t* ptr(int i, uint32_t ko) const {
    const int64_t bank = ((alt_mask >> i) & 1u) ? alt_delta : 0;
    return src + bank + (off[i] + ko);
  }
};

template <int S, class Plan>
AKAS_DEV void copy_piece(const Plan& p, int i, uint32_t ko) {
  __builtin_amdgcn_global_load_lds((const void*)p.ptr(i, ko),
                                   (lds_void*)(stage_base<S>() + (p.blk0 + i) * 1024), 16, 0, 0);
}
template <int S, class Plan>
AKAS_DEV void copy_scales(const Plan& p, int kb) {
  if (p.scales)
    __builtin_amdgcn_global_load_lds((const void*)(p.as + (p.soff + kb)),
                                     (lds_void*)(stage_scales<S>() + (p.blk0 >> 3) * 64), 4, 0, 0);
}
template <int S, class Plan>
AKAS_DEV void copy_stage(const Plan& p, int kb) {
  const uint32_t ko = (uint32_t)kb * 128;
#pragma unroll
  for (int i = 0; i < 8; ++i) copy_piece<S>(p, i, ko);
  copy_scales<S>(p, kb);
}

struct Acc {
  v4f t[4][8];  // [m-tile][n-tile], lane: row l%16, columns 4*(l/16) .. +3
  AKAS_DEV void clear() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) t[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  }
};

// Multiply stage S into acc and stream k-block kb_next into stage 1-S.
//   PAIRED: odd n-tiles use weight scale ws1 (gate/up tiles interleaved
//   16 rows at a time), even n-tiles ws0.
//   LIVE: false when every output row or column of the wave's 64x128 tile
//   is past the matrix (a partial last tile); the wave then only issues its
//   copies, and the live waves have the LDS to themselves.
// Each n-tile's four products are folded right after their MFMAs: the fold
// waits for the MFMA results, and the other wave on the SIMD issues its
// MFMAs meanwhile (keeping the previous products in flight instead costs 16
// registers and measured no faster).
template <int S, bool PAIRED, bool LIVE, class Plan>
AKAS_DEV void multiply(const Plan& p, Acc& acc, int a_row0, int b_row0, float ws0, float ws1,
                       int lane, int kb_next) {
  const uint8_t* at = stage_base<S>();
  const uint8_t* bt = at + BM * 128;
  const uint32_t ko = (uint32_t)kb_next * 128;
  if constexpr (!LIVE) {
    if (!p.skip) copy_stage<1 - S>(p, kb_next);
    return;
  }
  v8i af[4];
  float c0[4], c1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    af[i] = fragment(at, a_row0 + 16 * i, lane);
    const float s = stage_scales<S>()[a_row0 + 16 * i + (lane & 15)];
    c0[i] = s * ws0;
    c1[i] = PAIRED ? s * ws1 : c0[i];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    copy_piece<1 - S>(p, j, ko);
    if (j == 0) copy_scales<1 - S>(p, kb_next);
    const v8i bf = fragment(bt, b_row0 + 16 * j, lane);
    v4f cur[4];
    // The wave issuing MFMAs goes first; its SIMD partner's LDS reads and
    // folds fill the gaps (measured 5-9% faster than equal priority).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = mfma_e4m3(bf, af[i]);
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float c = (j & 1) ? c1[i] : c0[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc.t[i][j][e] = __builtin_fmaf(cur[i][e], c, acc.t[i][j][e]);
    }
  }
}

// Main loop over k-blocks [kb0, kb1).  ws(kb) returns (ws0, ws1) of a k-block
// as a float2.  Every stage refills the other one with k-block
// min(kb + 1, kb1 - 1): the refetch of the last block lands in a stage that
// is never read again, and the closing barrier waits for it.
template <bool PAIRED, bool LIVE, class Plan, class WS>
AKAS_DEV void run_(const Plan& p, Acc& acc, int a_row0, int b_row0, int kb0, int kb1, int lane, WS ws) {
  if (LIVE || !p.skip) copy_stage<0>(p, kb0);
  float2 wcur = ws(kb0);
  __syncthreads();
  const int last = kb1 - 1;
  for (int kb = kb0; kb < kb1; kb += 2) {
    float2 wnext = ws(min(kb + 1, last));
    multiply<0, PAIRED, LIVE>(p, acc, a_row0, b_row0, wcur.x, wcur.y, lane, min(kb + 1, last));
    __syncthreads();
    if (kb + 1 < kb1) {
      wcur = wnext;
      wnext = ws(min(kb + 2, last));
      multiply<1, PAIRED, LIVE>(p, acc, a_row0, b_row0, wcur.x, wcur.y, lane, min(kb + 2, last));
      __syncthreads();
      wcur = wnext;
    }
  }
}
template <bool PAIRED, class Plan, class WS>
AKAS_DEV void run(const Plan& p, Acc& acc, int a_row0, int b_row0, int kb0, int kb1, int lane, WS ws,
                  bool live) {
  if (live)  // wave-uniform: two loops, so the live one keeps its registers
    run_<PAIRED, true>(p, acc, a_row0, b_row0, kb0, kb1, lane, ws);
  else
    run_<PAIRED, false>(p, acc, a_row0, b_row0, kb0, kb1, lane, ws);
}

AKAS_DEV uint32_t pack2(float lo, float hi, int dt) {
  return dt == AKAS_DTYPE_BF16 ? f32x2_to_bf16x2(lo, hi) : f32x2_to_f16x2(lo, hi);
}

// Write the wave's 64x128 tile.  16-bit outputs go through a per-wave 16 KB
// LDS region (256-byte rows, 16-byte chunks XOR row) so that global stores
// are full 16-byte lanes along rows; f32 outputs store 4 columns per lane
// directly.  row_ok(r) / out_row(r) map a wave-local row to validity and to
// the output element offset of its first column (columns are contiguous).
// Must follow the main loop's closing barrier.
template <int OUT, class RowOk, class OutRow>
AKAS_DEV void store_tile(const Acc& acc, void* out, int wave, int lane, RowOk row_ok, OutRow out_row) {
  if constexpr (OUT == AKAS_DTYPE_F32) {
    float* o = reinterpret_cast<float*>(out);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * i + (lane & 15);
      if (!row_ok(r)) continue;
      const int64_t base = out_row(r);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int col = 16 * j + 4 * (lane >> 4);
        *reinterpret_cast<float4*>(o + base + col) = float4{acc.t[i][j][0], acc.t[i][j][1], acc.t[i][j][2], acc.t[i][j][3]};
      }
    }
  } else {
    uint8_t* region = (wave < 4 ? stage0 : stage1) + (wave & 3) * 16384;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = 16 * i + (lane & 15);
        const int col = 16 * j + 4 * (lane >> 4);
        uint2 v;
        v.x = pack2(acc.t[i][j][0], acc.t[i][j][1], OUT);
        v.y = pack2(acc.t[i][j][2], acc.t[i][j][3], OUT);
        *reinterpret_cast<uint2*>(region + r * 256 + (((col >> 3) ^ (r & 15)) << 4) + (col & 7) * 2) = v;
      }
    __syncthreads();
    uint16_t* o = reinterpret_cast<uint16_t*>(out);
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int r = it * 4 + (lane >> 4), ch = lane & 15;
      const u32x4 v = *reinterpret_cast<const u32x4*>(region + r * 256 + ((ch ^ (r & 15)) << 4));
      if (row_ok(r)) *reinterpret_cast<u32x4*>(o + out_row(r) + ch * 8) = v;
    }
  }
}

// store_tile for a wave whose row r (0..63) goes to element offset
// first + r * ldo and exists when r < rows: each lane's address is formed
// once and advanced by a constant stride, instead of once per store.  The
// 16-bit path stages through the wave's own LDS region (as store_tile), so
// only the wave's own order matters there: its LDS accesses complete in
// issue order, and the fence keeps the compiler from moving the reads above
// the writes.  Must follow the main loop's closing barrier.
template <int OUT>
AKAS_DEV void store_tile_rows(const Acc& acc, void* out, int wave, int lane, int rows, int64_t first, int64_t ldo) {
  if constexpr (OUT == AKAS_DTYPE_F32) {
    float* o = reinterpret_cast<float*>(out) + first + (int64_t)(lane & 15) * ldo + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (16 * i + (lane & 15) < rows) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<float4*>(o + 16 * j) =
              float4{acc.t[i][j][0], acc.t[i][j][1], acc.t[i][j][2], acc.t[i][j][3]};
      }
      o += 16 * ldo;
    }
  } else {
    uint8_t* region = (wave < 4 ? stage0 : stage1) + (wave & 3) * 16384;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = 16 * i + (lane & 15);
        const int col = 16 * j + 4 * (lane >> 4);
        uint2 v;
        v.x = pack2(acc.t[i][j][0], acc.t[i][j][1], OUT);
        v.y = pack2(acc.t[i][j][2], acc.t[i][j][3], OUT);
        *reinterpret_cast<uint2*>(region + r * 256 + (((col >> 3) ^ (r & 15)) << 4) + (col & 7) * 2) = v;
      }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int ch = lane & 15;
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + first + (int64_t)(lane >> 4) * ldo + ch * 8;
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int r = it * 4 + (lane >> 4);
      const u32x4 v = *reinterpret_cast<const u32x4*>(region + r * 256 + ((ch ^ (r & 15)) << 4));
      if (r < rows) *reinterpret_cast<u32x4*>(o) = v;
      o += 4 * ldo;
    }
  }
}

}  // namespace dma
}  // namespace akas
