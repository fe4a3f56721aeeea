// Tile engine shared by the dense and the grouped (expert) FP8 GEMMs.
//
// C[m, n] = sum_kb ( A_kb[m, :] . B_kb[n, :] ) * as[m, kb] * ws[n / 128, kb]
//
// A (activation codes) and B (weight codes) are both K-contiguous, so both
// feed the 16x16x128 FP8 MFMA with the same per-lane 32-byte k slices.  One
// MFMA covers exactly one 128-deep scale block: each block's partial product
// is formed in a fresh accumulator and folded into the running f32 total with
// one FMA by as[m]*ws (the reference's per-tile clear_accum + scale epilogue,
// src/akas/ops/linear/cuda.py:302-332).
//
// Workgroup tile BM x BN x 128, two LDS stages, global->register->LDS
// prefetch of the next k-block while the current one is multiplied.  LDS rows
// are 128 bytes with the 16-byte chunk index XOR-swizzled by
// (row & 7) ^ ((row >> 3) & 1): the 16 rows x 16 bytes that one quarter-wave
// of a fragment's ds_read_b128 reads then fall on 16 distinct 16-byte bank
// groups of the 256-byte-wide LDS (measured conflict-free with
// SQ_LDS_BANK_CONFLICT; (row >> 1) & 7 and row & 7 both conflict 2-way).  The
// swizzle depends on row % 16 only, so fragment addresses of tiles 16 rows
// apart differ by a constant and fold into the instruction offset.
#pragma once

#include "common.h"

namespace akas {

AKAS_DEV int lds_off(int row, int chunk) { return row * 128 + ((chunk ^ ((row & 7) ^ ((row >> 3) & 1))) << 4); }

// Staging plan: every thread moves CA chunks of the A tile and CB chunks of
// the B tile per k-block.  Thread t owns chunk column (t % 8) of rows
// t/8 + i*(THREADS/8); with THREADS >= 128 the swizzle term of those rows is
// the same for all i, so LDS destinations are dst0 + i*(THREADS/8)*128.
// A rows are gathered (one 32-bit offset per chunk); B rows are affine (one
// offset and a row step).  Offsets are relative to uniform base pointers, so
// the loads use scalar-base addressing with one VGPR per address.  Rows past the end of an operand are clamped to a valid row
// by the caller: their products land in rows/columns that are never stored
// or carry a zero scale, so no branch is needed in the copy loop.
template <int BM, int BN, int THREADS>
struct StagePlan {
  static constexpr int RSTEP = THREADS / 8;
  // A_PART: fewer A rows than thread rows (a 16-row tile on 256 threads):
  // the threads of the first BM rows move one A chunk each, the others none.
  static constexpr bool A_PART = BM < RSTEP;
  static constexpr int CA = A_PART ? 1 : BM / RSTEP;
  static constexpr int CB = BN / RSTEP;
  static_assert((BM % RSTEP == 0 || (A_PART && RSTEP % BM == 0)) && BN % RSTEP == 0,
                "tile rows must divide the thread rows");
  static_assert(THREADS >= 128, "swizzle invariance needs >= 16 thread rows");
  const uint8_t* a_base;  // uniform A base
  const uint8_t* b_base;  // uniform B base
  uint32_t a_off[CA];     // per-chunk A byte offset (k-block 0)
  uint32_t b_off;         // B byte offset of this thread's first row (k-block 0)
  uint32_t b_step;        // bytes between this thread's successive B rows
  int dst0;               // LDS offset of this thread's first chunk
  bool a_live = true;     // this thread moves A chunks (always unless A_PART)

  // Staging registers are kept in two small arrays (A chunks, B chunks):
  // one 128-byte array of uint4 is past what the alloca promotion keeps in
  // registers and would be placed in scratch.
  AKAS_DEV void fetch_a(int kb, u32x4 (&ra)[CA]) const {
    const uint32_t ko = (uint32_t)kb * kBlock;
#pragma unroll
    for (int i = 0; i < CA; ++i)
      if (!A_PART || a_live) ra[i] = *reinterpret_cast<const u32x4*>(a_base + (a_off[i] + ko));
  }
  AKAS_DEV void fetch_b(int kb, u32x4 (&rb)[CB]) const {
    const uint32_t ko = (uint32_t)kb * kBlock;
#pragma unroll
    for (int j = 0; j < CB; ++j)
      rb[j] = *reinterpret_cast<const u32x4*>(b_base + (b_off + j * b_step + ko));
  }
  AKAS_DEV void fetch(int kb, u32x4 (&ra)[CA], u32x4 (&rb)[CB]) const {
    fetch_a(kb, ra);
    fetch_b(kb, rb);
  }
  AKAS_DEV void stash(uint8_t* stage, const u32x4 (&ra)[CA], const u32x4 (&rb)[CB]) const {
#pragma unroll
    for (int i = 0; i < CA; ++i)
      if (!A_PART || a_live) *reinterpret_cast<u32x4*>(stage + dst0 + i * RSTEP * 128) = ra[i];
#pragma unroll
    for (int j = 0; j < CB; ++j)
      *reinterpret_cast<u32x4*>(stage + BM * 128 + dst0 + j * RSTEP * 128) = rb[j];
  }
};

// Per-wave accumulator tile: MT x NT MFMA tiles of 16x16 f32.
template <int MT, int NT>
struct Acc {
  v4f t[MT][NT];
  AKAS_DEV void clear() {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) t[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  }
};

// Load one MFMA operand fragment (16 rows x 128 k) for this lane from LDS.
AKAS_DEV v8i lds_fragment(const uint8_t* tile, int row0, int lane) {
  const int row = row0 + (lane & 15), g = lane >> 4;
  const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + lds_off(row, 2 * g));
  const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + lds_off(row, 2 * g + 1));
  v8i f;
  f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
  f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
  return f;
}

// Multiply one k-block held in LDS and fold it into acc.
//   a_tile/b_tile: stage bases; a_row0/b_row0: this wave's first tile rows;
//   as_stage: BM activation scales of the stage; ws0: this wave's weight scale
//   (PAIRED: ws0 scales even n-tiles, ws1 odd n-tiles -- gate and up tiles
//   interleaved 16 rows at a time).
// acc += P * (as[m] * ws) with one fresh MFMA product P per 16x16 tile.  The
// scale FMAs of n-tile j-1 are issued while the MFMAs of n-tile j run, so MT
// independent products are always in flight.
template <int MT, int NT, bool PAIRED = false>
AKAS_DEV void mma_stage(Acc<MT, NT>& acc, const uint8_t* a_tile, const uint8_t* b_tile,
                        const float* as_stage, int a_row0, int b_row0, float ws0, int lane,
                        float ws1 = 0.f) {
  v8i af[MT];
  float c0[MT][4], c1[MT][PAIRED ? 4 : 1];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    af[i] = lds_fragment(a_tile, a_row0 + 16 * i, lane);
    const float4 s4 = *reinterpret_cast<const float4*>(as_stage + a_row0 + 16 * i + 4 * (lane >> 4));
    c0[i][0] = s4.x * ws0; c0[i][1] = s4.y * ws0; c0[i][2] = s4.z * ws0; c0[i][3] = s4.w * ws0;
    if constexpr (PAIRED) {
      c1[i][0] = s4.x * ws1; c1[i][1] = s4.y * ws1; c1[i][2] = s4.z * ws1; c1[i][3] = s4.w * ws1;
    }
  }
  v4f prev[MT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const v8i bf = lds_fragment(b_tile, b_row0 + 16 * j, lane);
    v4f cur[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) cur[i] = mfma_e4m3(af[i], bf);
    if (j > 0) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float c = (PAIRED && ((j - 1) & 1)) ? c1[i][PAIRED ? e : 0] : c0[i][e];
          acc.t[i][j - 1][e] = __builtin_fmaf(prev[i][e], c, acc.t[i][j - 1][e]);
        }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) prev[i] = cur[i];
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = (PAIRED && ((NT - 1) & 1)) ? c1[i][PAIRED ? e : 0] : c0[i][e];
      acc.t[i][NT - 1][e] = __builtin_fmaf(prev[i][e], c, acc.t[i][NT - 1][e]);
    }
}

// Store an accumulator element in the output dtype (compile-time).
template <int DT>
AKAS_DEV void store_out(void* out, int64_t i, float v) {
  if constexpr (DT == AKAS_DTYPE_F32)
    reinterpret_cast<float*>(out)[i] = v;
  else if constexpr (DT == AKAS_DTYPE_BF16)
    reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
  else
    reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_f16_bits(v);
}

// Four consecutive output elements in one vector store (16 bytes of f32, 8
// of f16/bf16); `i` must keep the store aligned.
template <int DT>
AKAS_DEV void store_out4(void* out, int64_t i, const v4f& v) {
  if constexpr (DT == AKAS_DTYPE_F32) {
    *reinterpret_cast<v4f*>(reinterpret_cast<float*>(out) + i) = v;
  } else {
    uint2 q;
    if constexpr (DT == AKAS_DTYPE_BF16) {
      q.x = f32x2_to_bf16x2(v[0], v[1]);
      q.y = f32x2_to_bf16x2(v[2], v[3]);
    } else {
      q.x = f32x2_to_f16x2(v[0], v[1]);
      q.y = f32x2_to_f16x2(v[2], v[3]);
    }
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + i) = q;
  }
}

}  // namespace akas
