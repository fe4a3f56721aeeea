// Expert routing, stable route compaction, tile maps, expert packing, the
// expert-row SwiGLU and the weighted top-k combine for gfx950.
//
// Everything that fixes a permutation (top-k ids, routes, tile maps, pack
// offsets) is integer or exact-compare work and is bit-exact by construction:
// selection compares IEEE float32 scores with lowest-index tie breaking and
// the route compaction is an ordered block scan, never an atomic cursor.
#include "common.h"
#include "moe_launch.h"
#include "quant_group.h"

namespace akas {

// ---------------------------------------------------------------------------
// routers: one wave per token row
// ---------------------------------------------------------------------------

// (score, index) pairs: the larger score wins, ties -> the lower index.  One
// DPP step combines each lane with the lane CTRL selects.
template <int CTRL>
AKAS_DEV void argmax_step(float& s, int& idx) {
  const float os = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), CTRL, 0xF, 0xF, true));
  const int oi = __builtin_amdgcn_update_dpp(0, idx, CTRL, 0xF, 0xF, true);
  // Selects over non-short-circuit tests: an if, or || and &&, compiled
  // to exec-mask branches that made each rank of the top-k several times
  // longer.
  const bool take = (os > s) | ((os == s) & (oi < idx));
  s = take ? os : s;
  idx = take ? oi : idx;
}

// Arg-max over a 16-lane DPP row: quad swaps, then half-row and row mirrors.
AKAS_DEV void row_argmax(float& s, int& idx) {
  argmax_step<0xB1>(s, idx);   // quad_perm [1,0,3,2]
  argmax_step<0x4E>(s, idx);   // quad_perm [2,3,0,1]
  argmax_step<0x141>(s, idx);  // row_half_mirror: lane i <- 7 - i within 8 lanes
  argmax_step<0x140>(s, idx);  // row_mirror: lane i <- 15 - i within 16 lanes
}

// Arg-max across the wave: the four row results are read out as uniform values
// and combined in order; every lane returns the same pair.
AKAS_DEV void wave_argmax(float& s, int& idx) {
  row_argmax(s, idx);
  float bs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
  int bi = __builtin_amdgcn_readlane(idx, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const float os = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 16 * r));
    const int oi = __builtin_amdgcn_readlane(idx, 16 * r);
    const bool take = (os > bs) | ((os == bs) & (oi < bi));
    bs = take ? os : bs;
    bi = take ? oi : bi;
  }
  s = bs;
  idx = bi;
}

// Bitwise OR over a 16-lane DPP row (same steps as row_argmax).
template <int CTRL>
AKAS_DEV uint32_t or_step(uint32_t v) {
  return v | (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

constexpr int kMaxExpertSlots = 16;  // experts <= 64 * 16 = 1024
constexpr int kMaxTop = 32;

// Iterative top-k by maximum with lowest-index ties
// (src/akas/ops/moe/kernel.py:176-193, :467-483), one wave per row, lane l
// holding experts l, l + 64, ... (SLOTS per lane: experts <= 64 * SLOTS).
// BF16: the logits are rounded to bf16 on load (the block-fp8 "router" kind,
// src/akas/ops/moe/cuda.py:2011-2050).  The chosen expert's value is read out of
// its owner lane's registers (no load after the arg-max), and lane `rank`
// keeps rank's value and id, so the top-k lives in registers without a
// per-rank array.  Weights: the rank-ordered sums of the reference.
// Rows 4 * block .. 4 * block + 3 (one per wave).
template <int SOFTMAX, int SLOTS, int BF16>
AKAS_DEV void router_rows(const float* __restrict__ logits, const float* __restrict__ bias,
                          int32_t* __restrict__ ids, float* __restrict__ weights, int64_t rows,
                          int experts, int top, float scale, int normalize, int block) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)block * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform per wave
  const float* l = logits + row * experts;
  // base: the value a chosen expert contributes (the logit, or its sigmoid);
  // score: base + bias, the selection key.
  //
  // Every slot's logit (and bias) load goes out before the first is used:
  // loads under a per-lane condition each waited for the one before (four
  // memory round trips in series at 256 experts).  Indices past the experts
  // read the last one and are masked below.
  float base[SLOTS], score[SLOTS], raw[SLOTS], braw[SLOTS];
  const int slots = (experts + 63) / 64;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int e = min(s * 64 + lane, experts - 1);
    raw[s] = l[e];
    braw[s] = bias ? bias[e] : 0.f;
  }
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int e = s * 64 + lane;
    float v = 0.f, sc = -__builtin_inff();
    if (s < slots && e < experts) {
      v = SOFTMAX ? (BF16 ? round_bf16(raw[s]) : raw[s]) : router_sigmoid(raw[s]);
      sc = v + braw[s];
    }
    base[s] = v;
    score[s] = sc;
  }
  bool valid[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) valid[s] = (s < slots) & (s * 64 + lane < experts);
  float mine = 0.f;
  int mine_id = 0;
  for (int rank = 0; rank < top; ++rank) {
    float best = -__builtin_inff();
    int bi = 0x7FFFFFFF;
    // slots ascend in expert index, so strict > keeps the lowest index on
    // ties (selects over non-short-circuit tests, as in argmax_step)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const bool take = valid[s] & ((score[s] > best) | (bi == 0x7FFFFFFF));
      best = take ? score[s] : best;
      bi = take ? s * 64 + lane : bi;
    }
    wave_argmax(best, bi);
    const int owner = bi & 63, slot = bi >> 6;  // uniform
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      v = s == slot ? base[s] : v;
      score[s] = ((s == slot) & (lane == owner)) ? -__builtin_inff() : score[s];
    }
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), owner));
    if (lane == rank) {
      mine = v;
      mine_id = bi;
    }
  }
  float w;
  if (SOFTMAX) {
    float peak = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), 0));
    for (int i = 1; i < top; ++i)
      peak = __builtin_fmaxf(peak, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), i)));
    const float ex = expf(mine - peak);
    float total = 0.f;
    for (int i = 0; i < top; ++i) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), i));
    w = __fdiv_rn(scale * ex, total);
  } else {
    float den = normalize ? 1e-6f : 1.0f;
    if (normalize)
      for (int i = 0; i < top; ++i) den += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), i));
    w = __fdiv_rn(mine * scale, den);
  }
  if (lane < top) {
    ids[row * top + lane] = mine_id;
    weights[row * top + lane] = w;
  }
}

template <int SOFTMAX, int SLOTS, int BF16>
__global__ __launch_bounds__(256) void router_kernel(const float* __restrict__ logits,
                                                     const float* __restrict__ bias,
                                                     int32_t* __restrict__ ids,
                                                     float* __restrict__ weights, int64_t rows,
                                                     int experts, int top, float scale,
                                                     int normalize) {
  router_rows<SOFTMAX, SLOTS, BF16>(logits, bias, ids, weights, rows, experts, top, scale,
                                    normalize, blockIdx.x);
}

// experts <= 64 and top <= 8: four rows per wave, sixteen lanes per row (one
// DPP row), each lane holding four consecutive experts.  A rank's arg-max is
// a four-way scan of the lane's scores plus four DPP steps over the row (quad
// swaps, then half-row and row mirrors); the chosen expert's value reaches
// every lane of the row by OR-ing bit patterns over the same steps (the other
// lanes contribute zero bits), so nothing waits on a load after the
// arg-max.  Per wave that is a short instruction stream, which is what the
// decode-sized router's latency is made of.  Selection rule and weight
// arithmetic are router_kernel's, so ids and weights are identical.
constexpr int kRowTop = 8;

template <int SOFTMAX, int BF16>
AKAS_DEV void router_row16(const float* __restrict__ logits, const float* __restrict__ bias,
                           int32_t* __restrict__ ids, float* __restrict__ weights, int64_t rows,
                           int experts, int top, float scale, int normalize, int64_t block) {
  const int lane = threadIdx.x & 63, l = lane & 15;
  const int64_t row = (block * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const bool live = row < rows;
  const float* lg = logits + (live ? row : 0) * experts;  // spare rows read row 0, never stored
  // base: the value a chosen expert contributes (the logit, or its sigmoid);
  // score: base + bias, the selection key.
  // (All four loads go out before the first is used, as in router_kernel.)
  float base[4], score[4], raw[4], braw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = min(l * 4 + i, experts - 1);
    raw[i] = lg[e];
    braw[i] = bias ? bias[e] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = l * 4 + i;
    float v = 0.f, sc = -__builtin_inff();
    if (e < experts) {
      v = SOFTMAX ? (BF16 ? round_bf16(raw[i]) : raw[i]) : router_sigmoid(raw[i]);
      sc = v + braw[i];
    }
    base[i] = v;
    score[i] = sc;
  }
  float chosen[kRowTop];
  int chosen_id[kRowTop];
#pragma unroll
  for (int rank = 0; rank < kRowTop; ++rank) {
    chosen[rank] = 0.f;
    chosen_id[rank] = 0;
    if (rank >= top) continue;
    float best = -__builtin_inff();
    int bi = 0x7FFFFFFF;
    // ascending expert index, so strict > keeps the lowest index on ties
    // (selects over non-short-circuit tests, as in argmax_step)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = l * 4 + i;
      const bool take = (e < experts) & ((score[i] > best) | (bi == 0x7FFFFFFF));
      best = take ? score[i] : best;
      bi = take ? e : bi;
    }
    row_argmax(best, bi);
    chosen_id[rank] = bi;
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool mine_e = l * 4 + i == bi;
      bits = mine_e ? __float_as_uint(base[i]) : bits;
      score[i] = mine_e ? -__builtin_inff() : score[i];
    }
    bits = or_step<0xB1>(bits);
    bits = or_step<0x4E>(bits);
    bits = or_step<0x141>(bits);
    bits = or_step<0x140>(bits);
    chosen[rank] = __uint_as_float(bits);
  }
  // Lane l of the row stores rank l.
  float mine = 0.f;
  int mine_id = 0;
#pragma unroll
  for (int i = 0; i < kRowTop; ++i)
    if (i == l) {
      mine = chosen[i];
      mine_id = chosen_id[i];
    }
  float w;
  if (SOFTMAX) {
    float peak = chosen[0];
#pragma unroll
    for (int i = 1; i < kRowTop; ++i)
      if (i < top) peak = __builtin_fmaxf(peak, chosen[i]);
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < kRowTop; ++i)
      if (i < top) total += expf(chosen[i] - peak);
    w = __fdiv_rn(scale * expf(mine - peak), total);
  } else {
    float den = normalize ? 1e-6f : 1.0f;
    if (normalize) {
#pragma unroll
      for (int i = 0; i < kRowTop; ++i)
        if (i < top) den += chosen[i];
    }
    w = __fdiv_rn(mine * scale, den);
  }
  if (live && l < top) {
    ids[row * top + l] = mine_id;
    weights[row * top + l] = w;
  }
}

template <int SOFTMAX, int BF16>
__global__ __launch_bounds__(256) void router_row16_kernel(const float* __restrict__ logits,
                                                           const float* __restrict__ bias,
                                                           int32_t* __restrict__ ids,
                                                           float* __restrict__ weights,
                                                           int64_t rows, int experts, int top,
                                                           float scale, int normalize) {
  router_row16<SOFTMAX, BF16>(logits, bias, ids, weights, rows, experts, top, scale, normalize,
                              blockIdx.x);
}

// The quantizer half of a router + quantizer launch: workgroups from
// `first_block` on quantize x row-major, 16 groups per workgroup and pass
// (the quantizer's grid-stride loop and quantize8, so the codes are the
// quantizer's).
template <int DT>
AKAS_DEV void quantize_tail(const void* __restrict__ x, uint8_t* __restrict__ codes,
                            float* __restrict__ scales, int64_t groups, int first_block) {
  const int lane16 = threadIdx.x & 15;
  const int64_t qblocks = (int64_t)gridDim.x - first_block;
  const int64_t first = (((int64_t)blockIdx.x - first_block) * blockDim.x + threadIdx.x) >> 4;
  const int64_t stride = (qblocks * blockDim.x) >> 4;
  for (int64_t g = first; g < groups; g += stride) {
    const int64_t base = g * kBlock + lane16 * 8;
    float v[8], sc;
    load8<DT>(x, base, v);
    const uint2 c = quantize8(v, sc);
    *reinterpret_cast<uint2*>(codes + base) = c;
    if (lane16 == 0) scales[g] = sc;
  }
}

// The MoE block's router and its input quantizer in one launch: the first
// router_blocks workgroups route 16 rows each (router_row16), the rest
// quantize x row-major, 16 groups per workgroup and pass (the quantizer's
// grid-stride loop, same quantize8, so the codes are the quantizer's).  The
// two halves share nothing; one launch instead of two at decode sizes.
template <int SOFTMAX, int DT>
__global__ __launch_bounds__(256) void router_quantize_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int32_t* __restrict__ ids,
    float* __restrict__ weights, int64_t rows, int experts, int top, float scale, int normalize,
    int router_blocks, const void* __restrict__ x, uint8_t* __restrict__ codes,
    float* __restrict__ scales, int64_t groups) {
  if ((int)blockIdx.x < router_blocks) {
    router_row16<SOFTMAX, 0>(logits, bias, ids, weights, rows, experts, top, scale, normalize,
                             blockIdx.x);
    return;
  }
  quantize_tail<DT>(x, codes, scales, groups, router_blocks);
}

// The shared-expert block's decode router (bf16-rounded logits, softmax over
// the top-k, weights normalized) and its input quantizer in one launch, as
// router_quantize_kernel: SLOTS 0 routes 16 rows per workgroup
// (router_row16, up to 64 experts and top 8), else 4 (router_rows).
template <int SLOTS, int DT>
__global__ __launch_bounds__(256) void decode_router_quantize_kernel(
    const float* __restrict__ logits, int32_t* __restrict__ ids, float* __restrict__ weights,
    int64_t rows, int experts, int top, int router_blocks, const void* __restrict__ x,
    uint8_t* __restrict__ codes, float* __restrict__ scales, int64_t groups) {
  if ((int)blockIdx.x < router_blocks) {
    if constexpr (SLOTS == 0)
      router_row16<1, 1>(logits, nullptr, ids, weights, rows, experts, top, 1.0f, 1, blockIdx.x);
    else
      router_rows<1, SLOTS, 1>(logits, nullptr, ids, weights, rows, experts, top, 1.0f, 1,
                               blockIdx.x);
    return;
  }
  quantize_tail<DT>(x, codes, scales, groups, router_blocks);
}

// ---------------------------------------------------------------------------
// quantized_routes: one 1024-thread workgroup per expert, ordered block scan
// over the rows (src/akas/ops/moe/kernel.py:121-151, cuda.py:2187-2322)
//
// A route names the (row, rank) entry row * ld + rank (ld = top for
// quantized_routes).  With ld = top + 1, one more workgroup (expert index
// `experts`) routes every active row at rank top: the shared expert of the
// shared-expert block, riding in the routed launches.  Null active: every
// row is active.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void routes_kernel(const int32_t* __restrict__ ids,
                                                      const int32_t* __restrict__ active,
                                                      int32_t* __restrict__ counts,
                                                      int32_t* __restrict__ routes, int64_t rows,
                                                      int top, int ld = 0) {
  __shared__ int wave_tot[16];
  const int e = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t* out = routes + (int64_t)e * rows;
  if (ld == 0) ld = top;
  const bool extra = e == (int)gridDim.x - 1 && ld > top;  // the rank-`top` expert
  int64_t base = 0;
  for (int64_t r0 = 0; r0 < rows; r0 += 1024) {
    const int64_t row = r0 + tid;
    // Up to 32 ranks, the row's matches are kept as a bit mask, so its ids
    // are read once (with its activity flag, in one round trip) for both
    // the count and the writes.
    int cnt = 0;
    uint32_t mask = 0;
    if (row < rows) {
      const bool act = !active || active[row] != 0;
      if (extra) {
        cnt = 1;
      } else if (top <= 32) {
        for (int k = 0; k < top; ++k) mask |= (uint32_t)(ids[row * top + k] == e) << k;
        cnt = __builtin_popcount(mask);
      } else {
        for (int k = 0; k < top; ++k) cnt += ids[row * top + k] == e;
      }
      if (!act) cnt = 0;
    }
    const int incl = wave_inclusive_scan(cnt, lane);
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int t = wave_tot[w];
      before += w < wave ? t : 0;
      total += t;
    }
    if (cnt) {
      int64_t pos = base + before + incl - cnt;
      if (extra) {
        if (pos < rows) out[pos] = (int32_t)(row * ld + top);
      } else if (top <= 32) {
        for (uint32_t m = mask; m; m &= m - 1) {
          if (pos < rows) out[pos] = (int32_t)(row * ld + __builtin_ctz(m));
          ++pos;
        }
      } else {
        for (int k = 0; k < top; ++k)
          if (ids[row * top + k] == e) {
            if (pos < rows) out[pos] = (int32_t)(row * ld + k);
            ++pos;
          }
      }
    }
    base += total;
    __syncthreads();
  }
  const int64_t used = base < rows ? base : rows;
  for (int64_t i = used + tid; i < rows; i += 1024) out[i] = -1;
  // counts never exceed the routes row length (only reachable with duplicate
  // ids in one row, which top-k selection never produces)
  if (tid == 0) counts[e] = (int32_t)used;
}

// top = 4: four consecutive rows per thread (one 16-byte load of their ids,
// one of their activity flags), 4096 rows per pass, and the next pass's loads
// in flight while this pass is scanned and written.  Routes come out in the
// same (row, rank) order as the generic kernel's.
__global__ __launch_bounds__(1024) void routes4_kernel(const int32_t* __restrict__ ids,
                                                       const int32_t* __restrict__ active,
                                                       int32_t* __restrict__ counts,
                                                       int32_t* __restrict__ routes, int64_t rows) {
  constexpr int RPT = 4, PASS = 1024 * RPT;
  __shared__ int wave_tot[16];
  const int e = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t* out = routes + (int64_t)e * rows;
  // rows past the end read row 0 (their flags are masked below)
  auto load = [&](int64_t r0, int4 (&id)[RPT], int4& act) {
    const int64_t row = r0 + (int64_t)tid * RPT;
    const int64_t safe = row + RPT <= rows ? row : 0;
#pragma unroll
    for (int i = 0; i < RPT; ++i) id[i] = reinterpret_cast<const int4*>(ids)[safe + i];
    act = *reinterpret_cast<const int4*>(active + safe);
  };
  int4 id[RPT], act, nid[RPT], nact;
  load(0, id, act);
  int64_t base = 0;
  for (int64_t r0 = 0; r0 < rows; r0 += PASS) {
    if (r0 + PASS < rows) load(r0 + PASS, nid, nact);
    const int64_t row = r0 + (int64_t)tid * RPT;
    const int a[RPT] = {act.x, act.y, act.z, act.w};
    uint32_t mask[RPT];
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const bool live = row + i < rows && a[i] != 0;
      const int4 v = id[i];
      mask[i] = live ? (uint32_t)(v.x == e) | ((uint32_t)(v.y == e) << 1) |
                           ((uint32_t)(v.z == e) << 2) | ((uint32_t)(v.w == e) << 3)
                     : 0u;
      cnt += __builtin_popcount(mask[i]);
    }
    const int incl = wave_inclusive_scan(cnt, lane);
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int t = wave_tot[w];
      before += w < wave ? t : 0;
      total += t;
    }
    int64_t pos = base + before + incl - cnt;
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if ((mask[i] >> k) & 1u) {
          if (pos < rows) out[pos] = (int32_t)((row + i) * 4 + k);
          ++pos;
        }
    base += total;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RPT; ++i) id[i] = nid[i];
    act = nact;
  }
  const int64_t used = base < rows ? base : rows;
  for (int64_t i = used + tid; i < rows; i += 1024) out[i] = -1;
  if (tid == 0) counts[e] = (int32_t)used;
}

// ---------------------------------------------------------------------------
// moe_groups (src/akas/ops/moe/cuda.py:1978-2008), the block-fp8 decode
// variant's route tables: one workgroup per (row, rank) group g of the
// flattened ids.  g owns its expert when no earlier group holds it; the owner
// records the expert and, for every row b, the rank at which b selected it
// (the last such rank), -1 elsewhere; every other group records -1s.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_groups_kernel(const int32_t* __restrict__ ids,
                                                         int32_t* __restrict__ experts,
                                                         int32_t* __restrict__ routes,
                                                         int64_t rows, int top) {
  const int64_t g = blockIdx.x;
  const int expert = ids[g];
  int earlier = 0;
  for (int64_t e = threadIdx.x; e < g; e += 256) earlier |= ids[e] == expert;
  const bool owner = !__syncthreads_or(earlier);
  if (threadIdx.x == 0) experts[g] = owner ? expert : -1;
  int32_t* out = routes + g * rows;
  for (int64_t b = threadIdx.x; b < rows; b += 256) {
    int rank = -1;
    if (owner)
      for (int j = 0; j < top; ++j)
        if (ids[b * top + j] == expert) rank = j;
    out[b] = rank;
  }
}

// ---------------------------------------------------------------------------
// per-expert tile prefix (shared by the tile map and the pack kernel)
// ---------------------------------------------------------------------------

// prefix[e] = sum_{e' < e} ceil(counts[e'] / tile) (* mult); prefix[E] = total.
// Computed by wave 0 into LDS; E <= 1024.
AKAS_DEV void tile_prefix(const int32_t* counts, int experts, int tile, int mult, int* prefix,
                          int lane) {
  int carry = 0;
  for (int e0 = 0; e0 <= experts; e0 += 64) {
    const int e = e0 + lane;
    const int c = e < experts ? counts[e] : 0;
    const int n = ((c > 0 ? c : 0) + tile - 1) / tile * mult;
    const int incl = wave_inclusive_scan(n, lane);
    if (e <= experts) prefix[e] = carry + incl - n;
    carry += __shfl(incl, 63, 64);
  }
}

// The expert e with prefix[e] <= p < prefix[e+1] (it is non-empty), for
// 0 <= p < prefix[experts]; binary search keeps prefix[lo] <= p < prefix[hi].
AKAS_DEV int find_owner(const int* prefix, int experts, int p) {
  int lo = 0, hi = experts;  // prefix[lo] <= p < prefix[hi] holds when p < total
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (prefix[mid] <= p)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// (src/akas/ops/moe/kernel.py:79-118)
__global__ __launch_bounds__(256) void tile_map_kernel(const int32_t* __restrict__ counts,
                                                       int32_t* __restrict__ tile_experts,
                                                       int32_t* __restrict__ tile_rows,
                                                       int experts, int capacity) {
  __shared__ int prefix[1025];
  const int layout = blockIdx.y;
  const int tile = 4 << layout;
  if (threadIdx.x < 64) tile_prefix(counts, experts, tile, 1, prefix, threadIdx.x);
  __syncthreads();
  const int total = prefix[experts];
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= capacity) return;
  int32_t ex = -1, tr = 0;
  if (p < total) {
    ex = find_owner(prefix, experts, p);
    tr = p - prefix[ex];
  }
  tile_experts[(int64_t)layout * capacity + p] = ex;
  tile_rows[(int64_t)layout * capacity + p] = tr;
}

// expert_pack: 16 packed rows per 256-thread workgroup, 16 threads per row.
// (src/akas/ops/moe/cuda.py:2423-2502, oracle validation.py:621-642)
__global__ __launch_bounds__(256) void pack_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ as,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ routes,
    uint8_t* __restrict__ packed, float* __restrict__ packed_scales,
    int32_t* __restrict__ expert_offsets, int64_t rows, int top, int experts, int64_t k,
    int align, int64_t packed_rows, int routed, int64_t x_rows) {
  __shared__ int prefix[1025];
  if (threadIdx.x < 64) tile_prefix(counts, experts, align, align, prefix, threadIdx.x);
  __syncthreads();
  const int total = prefix[experts];
  const int sub = threadIdx.x & 15;
  const int64_t p = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (p >= total || p >= packed_rows) return;
  const int e = find_owner(prefix, experts, (int)p);
  const int local = (int)(p - prefix[e]);
  const int c = counts[e];
  const int64_t kb = k / kBlock;
  if (local == 0 && sub == 0) expert_offsets[e] = prefix[e];
  uint8_t* dst = packed + p * k;
  float* dsts = packed_scales + p * kb;
  const int route = local < c && local < rows ? routes[(int64_t)e * rows + local] : -1;
  const int64_t src_row = route < 0 ? -1 : (routed ? (int64_t)route : (int64_t)(route / top));
  if (src_row >= 0 && src_row < x_rows) {
    const uint8_t* src = x + src_row * k;
    for (int64_t i = sub * 16; i < k; i += 256)
      *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(src + i);
    for (int64_t i = sub; i < kb; i += 16) dsts[i] = as[src_row * kb + i];
  } else {
    for (int64_t i = sub * 16; i < k; i += 256)
      *reinterpret_cast<uint4*>(dst + i) = make_uint4(0, 0, 0, 0);
    for (int64_t i = sub; i < kb; i += 16) dsts[i] = 1.0f;
  }
}

// swiglu_experts (src/akas/ops/activation/kernel.py:28-88)
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ g,
                                                     const void* __restrict__ u, int in_dtype,
                                                     void* __restrict__ out, int out_dtype,
                                                     int64_t rows, int64_t c, int parts,
                                                     int round_inputs, int round_dtype) {
  const int64_t n = rows * c;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / c, col = i % c;
    float gv, uv;
    if (parts > 1) {
      gv = 0.f;
      uv = 0.f;
      for (int q = 0; q < parts; ++q) {
        gv += load_elem(g, (row * parts + q) * c + col, in_dtype);
        uv += load_elem(u, (row * parts + q) * c + col, in_dtype);
      }
    } else {
      gv = load_elem(g, i, in_dtype);
      uv = load_elem(u, i, in_dtype);
    }
    if (round_inputs) {
      gv = round_to(gv, round_dtype);
      uv = round_to(uv, round_dtype);
    }
    store_elem(out, i, swiglu_elem(gv, uv), out_dtype);
  }
}

// routed_combine (src/akas/ops/moe/kernel.py:206-267): 4 columns per thread.
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ experts,
                                                      int in_dtype,
                                                      const float* __restrict__ weights,
                                                      const int32_t* __restrict__ active,
                                                      float* __restrict__ out, int64_t rows,
                                                      int top, int64_t c) {
  const int64_t row = blockIdx.y;
  const int64_t col = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (col >= c) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (!active || active[row] != 0) {
    for (int k = 0; k < top; ++k) {
      const float wv = weights[row * top + k];
      const int64_t base = (row * top + k) * c + col;
      if (col + 4 <= c && in_dtype == AKAS_DTYPE_F32 && (c & 3) == 0) {
        const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(experts) + base);
        acc[0] = __builtin_fmaf(v.x, wv, acc[0]);
        acc[1] = __builtin_fmaf(v.y, wv, acc[1]);
        acc[2] = __builtin_fmaf(v.z, wv, acc[2]);
        acc[3] = __builtin_fmaf(v.w, wv, acc[3]);
      } else {
        for (int j = 0; j < 4; ++j)
          if (col + j < c) acc[j] = __builtin_fmaf(load_elem(experts, base + j, in_dtype), wv, acc[j]);
      }
    }
  }
  for (int j = 0; j < 4; ++j)
    if (col + j < c) out[row * c + col + j] = acc[j];
}

// Eight consecutive columns per thread with 16-byte loads (two for f32
// inputs), the loads of up to four ranks in flight before their folds; the
// fold order (rank 0 first, one fma per rank) is the generic kernel's, so the
// result is the same bit for bit.  c % 8 == 0 and 16-byte aligned rows.
//
// SHARED (moe_combine, src/akas/ops/moe/cuda.py:392-422): each rank's value
// is rounded to bf16 before its fold, and the shared expert enters as
// bf16(shared) / (1 + exp(-bf16(gate))) added after the ranks.
//
// ld: ranks per row of `experts` (top, or more when further ranks follow the
// combined ones); shared_ld: elements per row of `shared` (c, or ld * c for a
// shared expert stored as a rank of `experts`).
template <int DT, bool SHARED = false>
__global__ __launch_bounds__(256) void combine8_kernel(const void* __restrict__ experts,
                                                       const float* __restrict__ weights,
                                                       const int32_t* __restrict__ active,
                                                       float* __restrict__ out, int top,
                                                       int64_t c, const void* __restrict__ shared = nullptr,
                                                       int shared_dtype = 0,
                                                       const void* __restrict__ gate = nullptr,
                                                       int gate_dtype = 0, int ld = 0,
                                                       int64_t shared_ld = 0) {
  if (ld == 0) ld = top;
  if (shared_ld == 0) shared_ld = c;
  const int64_t row = blockIdx.y;
  const int64_t col = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (col >= c) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // SHARED: the gate and the shared row's eight values are requested before
  // the ranks' loads, as one or two 16-byte loads where the row is 16-byte
  // aligned (loaded element by element after the folds, each waited for the
  // one before).  The row's alignment is the same for every lane, since col
  // is a multiple of 8.
  uint32_t graw = 0;  // the gate's bits, widened after the folds
  u32x4 sraw[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
  bool svec = false;
  const int64_t sbase = row * shared_ld + col;
  if constexpr (SHARED) {
    graw = gate_dtype == AKAS_DTYPE_F32 ? reinterpret_cast<const uint32_t*>(gate)[row]
                                        : reinterpret_cast<const uint16_t*>(gate)[row];
    const bool f32 = shared_dtype == AKAS_DTYPE_F32;
    const uint8_t* at = reinterpret_cast<const uint8_t*>(shared) + sbase * (f32 ? 4 : 2);
    svec = (reinterpret_cast<uintptr_t>(at) & 15) == 0;
    if (svec) {
      const u32x4* src = reinterpret_cast<const u32x4*>(at);  // global, not flat, loads
      sraw[0] = src[0];
      if (f32) sraw[1] = src[1];
    }
  }
  // The contributions' loads are in bounds for every row, so they go out
  // without waiting for the row's flag, which only selects the result.
  {
    constexpr int U = 4;
    for (int k0 = 0; k0 < top; k0 += U) {
      u32x4 raw[U][DT == AKAS_DTYPE_F32 ? 2 : 1];
      float wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = min(k0 + u, top - 1);  // unconditional: a clamped rank is never folded
        wv[u] = weights[row * top + k];
        const int64_t base = (row * ld + k) * c + col;
        if constexpr (DT == AKAS_DTYPE_F32) {
          const u32x4* src = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(experts) + base);
          raw[u][0] = src[0];
          raw[u][1] = src[1];
        } else {
          raw[u][0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(experts) + base);
        }
      }
      // Rank by rank, each fold kept or discarded by a select rather than a
      // branch, so that all of the ranks' loads above go out before the first
      // fold waits for one (a branch per rank let the compiler sink each load
      // behind the previous rank's wait).
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool folds = k0 + u < top;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float v;
          if constexpr (DT == AKAS_DTYPE_F32)
            v = __uint_as_float(raw[u][j >> 2][j & 3]);
          else if constexpr (DT == AKAS_DTYPE_BF16)
            v = bf16_bits_to_f32((raw[u][0][j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
          else
            v = f16_bits_to_f32((raw[u][0][j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
          if constexpr (SHARED && DT != AKAS_DTYPE_BF16) v = round_bf16(v);
          const float f = __builtin_fmaf(v, wv[u], acc[j]);
          acc[j] = folds ? f : acc[j];
        }
      }
    }
  }
  if (active && active[row] == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  }
  if constexpr (SHARED) {
    const float gv = gate_dtype == AKAS_DTYPE_F32    ? __uint_as_float(graw)
                     : gate_dtype == AKAS_DTYPE_BF16 ? bf16_bits_to_f32(graw)
                                                      : f16_bits_to_f32(graw);
    const float g = round_bf16(gv);
    const float den = 1.0f + expf(-g);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float sv;
      if (!svec)
        sv = load_elem(shared, sbase + j, shared_dtype);
      else if (shared_dtype == AKAS_DTYPE_F32)
        sv = __uint_as_float(sraw[j >> 2][j & 3]);
      else if (shared_dtype == AKAS_DTYPE_BF16)
        sv = bf16_bits_to_f32((sraw[0][j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
      else
        sv = f16_bits_to_f32((sraw[0][j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
      acc[j] += __fdiv_rn(round_bf16(sv), den);
    }
  }
  float4* dst = reinterpret_cast<float4*>(out + row * c + col);
  dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

static inline bool float_dtype(int d) {
  return d == AKAS_DTYPE_F32 || d == AKAS_DTYPE_F16 || d == AKAS_DTYPE_BF16;
}

static inline int grid_for(int64_t n, int per = 256, int cap = 16384) {
  const int64_t want = (n + per - 1) / per;
  return (int)(want < cap ? (want > 0 ? want : 1) : cap);
}

// tile_capacity (src/akas/ops/moe/definition.py:9-16)
int64_t tile_capacity(int64_t rows, int64_t top, int64_t experts, int64_t block_m) {
  const int64_t routes = rows * top;
  const int64_t b = (routes + block_m - 1) / block_m + experts - 1;
  return routes < b ? routes : b;
}

bool valid_block(int m) { return m == 4 || m == 8 || m == 16 || m == 32 || m == 64 || m == 128; }

}  // namespace akas

using namespace akas;

// One row-per-16-lanes launch for <= 64 experts and top <= 8, else one wave
// per row with 4 or 16 expert slots per lane.
template <int SOFTMAX, int BF16>
static void launch_router(const float* logits, const float* bias, int32_t* ids, float* weights,
                          int64_t r, int experts, int top, float scale, int normalize,
                          hipStream_t s) {
  if (experts <= 64 && top <= kRowTop)
    router_row16_kernel<SOFTMAX, BF16><<<(int)((r + 15) / 16), 256, 0, s>>>(
        logits, bias, ids, weights, r, experts, top, scale, normalize);
  else if (experts <= 256)
    router_kernel<SOFTMAX, 4, BF16><<<(int)((r + 3) / 4), 256, 0, s>>>(
        logits, bias, ids, weights, r, experts, top, scale, normalize);
  else
    router_kernel<SOFTMAX, kMaxExpertSlots, BF16><<<(int)((r + 3) / 4), 256, 0, s>>>(
        logits, bias, ids, weights, r, experts, top, scale, normalize);
}

static int check_router(const float* logits, int32_t* ids, float* weights, int64_t r,
                        int experts, int top) {
  if (r < 0 || experts < 1 || experts > 64 * kMaxExpertSlots || top < 1 || top > experts ||
      top > kMaxTop || (r + 3) / 4 > 0x7FFFFFFF)
    return AKAS_ERR_GEOMETRY;
  if (r > 0 && (!logits || !ids || !weights)) return AKAS_ERR_NULL;
  return AKAS_OK;
}

// Launches run by the grouped expert kernels' entry points as well (declared
// in moe_launch.h); the arguments are checked by the entry points.
namespace akas {

int launch_decode_router_quantize(const float* logits, int32_t* ids, float* weights, int64_t r,
                                  int experts, int top, const void* x, int x_dtype,
                                  uint8_t* codes, float* scales, int64_t k, hipStream_t s) {
  const int st = check_router(logits, ids, weights, r, experts, top);
  if (st != AKAS_OK || r == 0) return st;
  if (k <= 0 || k % kBlock) return AKAS_ERR_GEOMETRY;
  if (!x || !codes || !scales) return AKAS_ERR_NULL;
  const bool row16 = experts <= 64 && top <= kRowTop;
  const int64_t groups = r * (k / kBlock);
  const int64_t rblocks = row16 ? (r + 15) / 16 : (r + 3) / 4, want = (groups + 15) / 16;
  const int64_t qblocks = want < 8192 ? want : 8192;
  if (rblocks + qblocks > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  const dim3 grid((unsigned)(rblocks + qblocks));
  auto go = [&](auto SL, auto XD) {
    decode_router_quantize_kernel<decltype(SL)::value, decltype(XD)::value><<<grid, 256, 0, s>>>(
        logits, ids, weights, r, experts, top, (int)rblocks, x, codes, scales, groups);
  };
  auto by_x = [&](auto SL) {
    switch (x_dtype) {
      case AKAS_DTYPE_F32: go(SL, DtypeTag<AKAS_DTYPE_F32>{}); break;
      case AKAS_DTYPE_F16: go(SL, DtypeTag<AKAS_DTYPE_F16>{}); break;
      default: go(SL, DtypeTag<AKAS_DTYPE_BF16>{});
    }
  };
  if (row16)
    by_x(DtypeTag<0>{});
  else if (experts <= 256)
    by_x(DtypeTag<4>{});
  else
    by_x(DtypeTag<kMaxExpertSlots>{});
  return AKAS_OK;
}

void launch_quantized_routes(const int32_t* ids, const int32_t* active, int32_t* counts,
                             int32_t* routes, int64_t r, int experts, int top, hipStream_t s) {
  // routes4_kernel's first pass loads ids[0..15] and active[0..3]
  // unconditionally, so it needs at least four rows and the flags; an empty
  // batch takes the generic kernel, which only writes counts[e] = 0.
  if (top == 4 && r >= 4 && r % 4 == 0 && active &&
      reinterpret_cast<uintptr_t>(active) % 16 == 0 && reinterpret_cast<uintptr_t>(ids) % 16 == 0)
    routes4_kernel<<<experts, 1024, 0, s>>>(ids, active, counts, routes, r);
  else
    routes_kernel<<<experts, 1024, 0, s>>>(ids, active, counts, routes, r, top);
}

void launch_routes_with_shared(const int32_t* ids, int32_t* counts, int32_t* routes, int64_t r,
                               int experts, int top, hipStream_t s) {
  routes_kernel<<<experts + 1, 1024, 0, s>>>(ids, nullptr, counts, routes, r, top, top + 1);
}

void launch_shared_rank_combine(const uint16_t* contributions, const float* weights,
                                const void* gate, int gate_dtype, float* out, int64_t r, int top,
                                int64_t c, hipStream_t s) {
  const int ld = top + 1;
  for (int64_t r0 = 0; r0 < r; r0 += 65535) {
    const int64_t rr = r - r0 < 65535 ? r - r0 : 65535;
    const uint16_t* ex = contributions + r0 * ld * c;
    const char* ga = reinterpret_cast<const char*>(gate) + r0 * (gate_dtype == AKAS_DTYPE_F32 ? 4 : 2);
    dim3 grid((unsigned)((c / 8 + 255) / 256), (unsigned)rr);
    combine8_kernel<AKAS_DTYPE_BF16, true><<<grid, 256, 0, s>>>(
        ex, weights + r0 * top, nullptr, out + r0 * c, top, c, ex + (int64_t)top * c,
        AKAS_DTYPE_BF16, ga, gate_dtype, ld, (int64_t)ld * c);
  }
}

}  // namespace akas

extern "C" int akas_biased_router(const float* logits, const float* bias, int32_t* ids,
                                  float* weights, int64_t r, int experts, int top, float scale,
                                  int normalize, void* stream) {
  const int st = check_router(logits, ids, weights, r, experts, top);
  if (st != AKAS_OK || r == 0) return st;
  launch_router<0, 0>(logits, bias, ids, weights, r, experts, top, scale, normalize,
                      reinterpret_cast<hipStream_t>(stream));
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_biased_softmax_router(const float* logits, const float* bias, int32_t* ids,
                                          float* weights, int64_t r, int experts, int top,
                                          float scale, void* stream) {
  const int st = check_router(logits, ids, weights, r, experts, top);
  if (st != AKAS_OK || r == 0) return st;
  launch_router<1, 0>(logits, bias, ids, weights, r, experts, top, scale, 1,
                      reinterpret_cast<hipStream_t>(stream));
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_router(const float* logits, int32_t* ids, float* weights, int64_t r,
                           int experts, int top, void* stream) {
  const int st = check_router(logits, ids, weights, r, experts, top);
  if (st != AKAS_OK || r == 0) return st;
  launch_router<1, 1>(logits, nullptr, ids, weights, r, experts, top, 1.0f, 1,
                      reinterpret_cast<hipStream_t>(stream));
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_router_quantize(const float* logits, const float* bias, int32_t* ids,
                                    float* weights, int64_t r, int experts, int top, float scale,
                                    int softmax, int normalize, const void* x, int x_dtype,
                                    uint8_t* codes, float* scales, int64_t k, void* stream) {
  int st = check_router(logits, ids, weights, r, experts, top);
  if (st != AKAS_OK) return st;
  if (experts > 64 || top > kRowTop || k <= 0 || k % kBlock) return AKAS_ERR_GEOMETRY;
  if (x_dtype != AKAS_DTYPE_F32 && x_dtype != AKAS_DTYPE_F16 && x_dtype != AKAS_DTYPE_BF16)
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !codes || !scales) return AKAS_ERR_NULL;
  const int64_t groups = r * (k / kBlock);
  const int64_t rblocks = (r + 15) / 16, want = (groups + 15) / 16;
  const int64_t qblocks = want < 8192 ? want : 8192;
  if (rblocks + qblocks > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(rblocks + qblocks));
  auto go = [&](auto SM, auto XD) {
    router_quantize_kernel<decltype(SM)::value, decltype(XD)::value><<<grid, 256, 0, s>>>(
        logits, bias, ids, weights, r, experts, top, scale, normalize, (int)rblocks, x, codes,
        scales, groups);
  };
  auto by_x = [&](auto SM) {
    switch (x_dtype) {
      case AKAS_DTYPE_F32: go(SM, DtypeTag<AKAS_DTYPE_F32>{}); break;
      case AKAS_DTYPE_F16: go(SM, DtypeTag<AKAS_DTYPE_F16>{}); break;
      default: go(SM, DtypeTag<AKAS_DTYPE_BF16>{});
    }
  };
  if (softmax)
    by_x(DtypeTag<1>{});
  else
    by_x(DtypeTag<0>{});
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_quantized_routes(const int32_t* ids, const int32_t* active, int32_t* counts,
                                     int32_t* routes, int64_t r, int experts, int top,
                                     void* stream) {
  if (r < 0 || experts < 1 || top < 1 || r * top > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  if (!counts || (r > 0 && (!ids || !active || !routes))) return AKAS_ERR_NULL;
  launch_quantized_routes(ids, active, counts, routes, r, experts, top,
                          reinterpret_cast<hipStream_t>(stream));
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_moe_groups(const int32_t* ids, int32_t* experts, int32_t* routes, int64_t r,
                               int top, void* stream) {
  if (r < 0 || top < 1 || r * top > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  if (r == 0) return AKAS_OK;
  if (!ids || !experts || !routes) return AKAS_ERR_NULL;
  moe_groups_kernel<<<(int)(r * top), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      ids, experts, routes, r, top);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_expert_tile_map(const int32_t* counts, int32_t* tile_experts,
                                    int32_t* tile_rows, int64_t r, int experts, int top,
                                    int max_block_m, void* stream) {
  if (r < 0 || experts < 1 || experts > 1024 || top < 1 || !valid_block(max_block_m))
    return AKAS_ERR_GEOMETRY;
  if (!counts || !tile_experts || !tile_rows) return AKAS_ERR_NULL;
  const int layouts = 32 - __builtin_clz((unsigned)max_block_m) - 2;
  const int64_t capacity = (r * top + 3) / 4 + experts;
  if (capacity > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  dim3 grid((unsigned)((capacity + 255) / 256), (unsigned)layouts);
  tile_map_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      counts, tile_experts, tile_rows, experts, (int)capacity);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_expert_pack(const uint8_t* x, const float* activation_scales,
                                const int32_t* counts, const int32_t* routes,
                                const int32_t* tile_experts, const int32_t* tile_offsets,
                                uint8_t* packed, float* packed_scales, int32_t* expert_offsets,
                                int64_t r, int top, int experts, int64_t k, int max_block_m,
                                int routed_input, void* stream) {
  (void)tile_experts;
  (void)tile_offsets;
  if (r < 1 || top < 1 || experts < 1 || experts > 1024 || k <= 0 || k % kBlock ||
      !valid_block(max_block_m))
    return AKAS_ERR_GEOMETRY;
  if (!x || !activation_scales || !counts || !routes || !packed || !packed_scales ||
      !expert_offsets)
    return AKAS_ERR_NULL;
  const int64_t packed_rows = tile_capacity(r, top, experts, max_block_m) * max_block_m;
  if (packed_rows > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  pack_kernel<<<(int)((packed_rows + 15) / 16), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      x, activation_scales, counts, routes, packed, packed_scales, expert_offsets, r, top, experts,
      k, max_block_m, packed_rows, routed_input, routed_input ? r * top : r);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_swiglu_experts(const void* g, const void* u, int input_dtype, void* out,
                                   int output_dtype, int64_t r, int top, int64_t c,
                                   int partitions, int round_inputs, int round_dtype,
                                   void* stream) {
  if (r < 0 || top < 1 || c <= 0 || partitions < 1) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(input_dtype) || !float_dtype(output_dtype) ||
      (round_inputs && !float_dtype(round_dtype)))
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!g || !u || !out) return AKAS_ERR_NULL;
  const int64_t rows = r * top;
  swiglu_kernel<<<grid_for(rows * c), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      g, u, input_dtype, out, output_dtype, rows, c, partitions, round_inputs, round_dtype);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_moe_combine(const void* experts, int input_dtype, const float* weights,
                                const void* shared, int shared_dtype, const void* gate,
                                int gate_dtype, float* out, int64_t r, int top, int64_t c,
                                void* stream) {
  if (r < 0 || top < 1 || c <= 0 || c % 8 || r > 65535 * 64) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(input_dtype) || !float_dtype(shared_dtype) || !float_dtype(gate_dtype))
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!experts || !weights || !shared || !gate || !out) return AKAS_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(experts) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return AKAS_ERR_GEOMETRY;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const size_t esz = input_dtype == AKAS_DTYPE_F32 ? 4 : 2;
  const size_t ssz = shared_dtype == AKAS_DTYPE_F32 ? 4 : 2;
  const size_t gsz = gate_dtype == AKAS_DTYPE_F32 ? 4 : 2;
  for (int64_t r0 = 0; r0 < r; r0 += 65535) {
    const int64_t rr = r - r0 < 65535 ? r - r0 : 65535;
    const char* ex = reinterpret_cast<const char*>(experts) + r0 * top * c * esz;
    const char* sh = reinterpret_cast<const char*>(shared) + r0 * c * ssz;
    const char* ga = reinterpret_cast<const char*>(gate) + r0 * gsz;
    dim3 grid((unsigned)((c / 8 + 255) / 256), (unsigned)rr);
    if (input_dtype == AKAS_DTYPE_F32)
      combine8_kernel<AKAS_DTYPE_F32, true><<<grid, 256, 0, s>>>(ex, weights + r0 * top, nullptr, out + r0 * c, top, c,
                                                                 sh, shared_dtype, ga, gate_dtype);
    else if (input_dtype == AKAS_DTYPE_BF16)
      combine8_kernel<AKAS_DTYPE_BF16, true><<<grid, 256, 0, s>>>(ex, weights + r0 * top, nullptr, out + r0 * c, top, c,
                                                                  sh, shared_dtype, ga, gate_dtype);
    else
      combine8_kernel<AKAS_DTYPE_F16, true><<<grid, 256, 0, s>>>(ex, weights + r0 * top, nullptr, out + r0 * c, top, c,
                                                                 sh, shared_dtype, ga, gate_dtype);
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_routed_combine(const void* experts, int input_dtype, const float* weights,
                                   const int32_t* active, float* out, int64_t r, int top,
                                   int64_t c, void* stream) {
  if (r < 0 || top < 1 || c <= 0 || r > 65535 * 64) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(input_dtype)) return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!experts || !weights || !out) return AKAS_ERR_NULL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const size_t esz = input_dtype == AKAS_DTYPE_F32 ? 4 : 2;
  const bool vec = c % 8 == 0 && reinterpret_cast<uintptr_t>(experts) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0;
  for (int64_t r0 = 0; r0 < r; r0 += 65535) {
    const int64_t rr = r - r0 < 65535 ? r - r0 : 65535;
    const char* ex = reinterpret_cast<const char*>(experts) + r0 * top * c * esz;
    const int32_t* act = active ? active + r0 : nullptr;
    if (vec) {
      dim3 grid((unsigned)((c / 8 + 255) / 256), (unsigned)rr);
      if (input_dtype == AKAS_DTYPE_F32)
        combine8_kernel<AKAS_DTYPE_F32><<<grid, 256, 0, s>>>(ex, weights + r0 * top, act, out + r0 * c, top, c);
      else if (input_dtype == AKAS_DTYPE_BF16)
        combine8_kernel<AKAS_DTYPE_BF16><<<grid, 256, 0, s>>>(ex, weights + r0 * top, act, out + r0 * c, top, c);
      else
        combine8_kernel<AKAS_DTYPE_F16><<<grid, 256, 0, s>>>(ex, weights + r0 * top, act, out + r0 * c, top, c);
    } else {
      dim3 grid((unsigned)((c + 1023) / 1024), (unsigned)rr);
      combine_kernel<<<grid, 256, 0, s>>>(ex, input_dtype, weights + r0 * top, act, out + r0 * c, rr, top, c);
    }
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}
