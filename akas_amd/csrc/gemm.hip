// Dense block-scaled FP8 linear for gfx950: small-M (decode) and LDS-tiled
// (prefill) MFMA kernels, split-K partials and the partition merge.
#include <atomic>
#include <mutex>

#include "device_info.h"
#include "gemm_core.h"
#include "gemm_dma.h"
#include "quant_group.h"

namespace akas {

struct DenseArgs {
  const uint8_t* a;   // activation codes [M, K]
  const float* as;    // activation scales [M, K/128]
  const uint8_t* w;   // weight codes [N, K]
  const void* ws;     // weight block scales [ceil(N/128), K/128]
  void* out;
  int64_t ldo;          // row stride of out, elements
  int64_t part_stride;  // element offset between partitions of out
  int M, N, K;
  int kb_per_part;      // k-blocks per partition
  int ws_dtype, out_dtype;
  const void* x;        // unquantized activations [M, K] (kernels that quantize while staging)
  int x_dtype;
};

// Logical tile id -> (tm, tn): groups of G m-tiles walked n-major so that a
// window of concurrently running workgroups shares both A and B tiles.
AKAS_DEV void grouped_tile(int id, int tiles_m, int tiles_n, int G, int& tm, int& tn) {
  const int per_group = G * tiles_n;
  const int group = id / per_group, first = group * G;
  const int gsize = min(tiles_m - first, G);
  const int local = id % per_group;
  tm = first + local % gsize;
  tn = local / gsize;
}

// ---------------------------------------------------------------------------
// LDS-tiled MFMA GEMM (prefill shapes and medium M)
//
// DEPTH k-blocks are in flight per workgroup in a register ring in front of
// the two LDS stages: at k-block kb the ring holds kb+1 .. kb+DEPTH, so the
// HBM latency of a load is covered by DEPTH k-block multiplies.  Decode-sized
// launches (few tiles, 16 k-blocks) need DEPTH 3-4; prefill tiles fill the
// GPU with enough workgroups that DEPTH 1 suffices.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WAVES_M, int WAVES_N, int DEPTH, int OUT, int SDT>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void dense_tiled_kernel(DenseArgs p) {
  constexpr int THREADS = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int MT = WM / 16, NT = WN / 16;
  static_assert(128 % WN == 0, "a wave's columns must stay inside one scale block");
  using Plan = StagePlan<BM, BN, THREADS>;
  constexpr int STAGE = (BM + BN) * 128;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];
  __shared__ __attribute__((aligned(16))) float lds_as[2][BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  int tm, tn;
  grouped_tile(id, tiles_m, tiles_n, 8, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int part = blockIdx.y;
  const int KB = p.K / kBlock;
  const int kb0 = part * p.kb_per_part, kb1 = kb0 + p.kb_per_part;

  Plan plan;
  {
    const int row = tid >> 3, ch = tid & 7;
#pragma unroll
    for (int i = 0; i < Plan::CA; ++i) {
      const int gm = min(m0 + row + i * Plan::RSTEP, p.M - 1);
      plan.a_off[i] = (uint32_t)gm * (uint32_t)p.K + ch * 16;
    }
    plan.a_base = p.a;
    plan.b_base = p.w;
    plan.b_off = (uint32_t)(n0 + row) * (uint32_t)p.K + ch * 16;
    plan.b_step = (uint32_t)Plan::RSTEP * (uint32_t)p.K;
    plan.dst0 = lds_off(row, ch);
  }
  // Rows past M read row M-1's scales; their outputs are never stored.
  const float* as_row = p.as + (int64_t)min(m0 + (tid < BM ? tid : 0), p.M - 1) * KB;

  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int a_row0 = wm * WM, b_row0 = wn * WN;
  const int wcol = n0 + b_row0;
  const int64_t ws_base = (int64_t)(wcol / kBlock) * KB;

  Acc<MT, NT> acc;
  acc.clear();
  // Ring slot = (A chunks, B chunks, activation scale, weight scale) of one
  // k-block.  Every global load, scales included, is issued DEPTH k-blocks
  // before its use: loads complete in issue order, so a scale fetched after
  // a prefetch would make the current multiply wait for that prefetch.
  u32x4 ring_a[DEPTH][Plan::CA], ring_b[DEPTH][Plan::CB];
  float ras[DEPTH], rws[DEPTH];
  const int last = kb1 - 1;
  // prologue: k-blocks kb0 .. kb0+DEPTH-1 in flight; stage 0 <- kb0
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    const int k = min(kb0 + d, last);
    plan.fetch(k, ring_a[d], ring_b[d]);
    ras[d] = as_row[k];
    rws[d] = load_scale_t<SDT>(p.ws, ws_base + k);
  }
  plan.stash(lds, ring_a[0], ring_b[0]);
  if (tid < BM) lds_as[0][tid] = ras[0];
  float ws_cur = rws[0];
  {
    const int k = min(kb0 + DEPTH, last);
    plan.fetch(k, ring_a[0], ring_b[0]);
    ras[0] = as_row[k];
    rws[0] = load_scale_t<SDT>(p.ws, ws_base + k);
  }
  __syncthreads();

  // Ring slot of k-block k is (k - kb0) % DEPTH; the loop body is expanded
  // DEPTH times with constant slot indices so the ring stays in registers.
  // Ring traffic is unconditional: past the last k-block it re-reads that
  // block into the idle stage, which is never consumed.
#define AKAS_RING_STEP(J)                                                            \
  if constexpr ((J) < DEPTH) {                                                       \
    const int k = kb + (J);                                                          \
    const int cur = (k - kb0) & 1;                                                   \
    if (k < kb1)                                                                     \
      mma_stage<MT, NT>(acc, lds + cur * STAGE, lds + cur * STAGE + BM * 128,        \
                        lds_as[cur], a_row0, b_row0, ws_cur, lane);                  \
    constexpr int ns = ((J) + 1) % DEPTH;                                            \
    plan.stash(lds + (cur ^ 1) * STAGE, ring_a[ns], ring_b[ns]);                     \
    if (tid < BM) lds_as[cur ^ 1][tid] = ras[ns];                                    \
    ws_cur = rws[ns];                                                                \
    const int kf = min(k + 1 + DEPTH, last);                                         \
    plan.fetch(kf, ring_a[ns], ring_b[ns]);                                          \
    ras[ns] = as_row[kf];                                                            \
    rws[ns] = load_scale_t<SDT>(p.ws, ws_base + kf);                            \
    __syncthreads();                                                                 \
  }
  for (int kb = kb0; kb < kb1; kb += DEPTH) {
    AKAS_RING_STEP(0)
    AKAS_RING_STEP(1)
    AKAS_RING_STEP(2)
    AKAS_RING_STEP(3)
    AKAS_RING_STEP(4)
    AKAS_RING_STEP(5)
  }
#undef AKAS_RING_STEP
  static_assert(DEPTH >= 1 && DEPTH <= 6, "prefetch depth 1..6");

  const int64_t obase = (int64_t)part * p.part_stride;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + a_row0 + 16 * i + 4 * (lane >> 4) + e;
        const int col = wcol + 16 * j + (lane & 15);
        if (row < p.M && col < p.N) store_out<OUT>(p.out, obase + (int64_t)row * p.ldo + col, acc.t[i][j][e]);
      }
}

// ---------------------------------------------------------------------------
// Decode-shape GEMM, 16 < M <= 256: split-K across the waves of a workgroup
//
// At these sizes the weights are the only operand that comes from HBM and
// the vector L1 is the other limit: at one workgroup per CU it passes about
// 100-120 GB/s per CU when each load instruction covers whole 128-byte
// lines (eight lanes per line), but only a third of that when sixteen rows
// share one instruction -- which is what loading straight into the MFMA
// operand order does.  So:
//   * A workgroup owns a BM x BN output tile; its four waves split the
//     k-range four ways.  Each wave stages its BN x 512-byte weight slice
//     (two rows of 512 contiguous bytes per load instruction) in a private
//     swizzled LDS region, requesting all of it up front, and reads MFMA
//     fragments back with conflict-free 16-byte LDS reads.
//   * Activations come either fragment-major (AF = 1: the quantizer in
//     fp8_linear writes 2 KB tiles in which one contiguous 1 KB load per half
//     is already in the MFMA lane order), or row-major (AF = 0, caller-owned
//     codes): four neighbouring lanes per row, moved to the MFMA lane order
//     with ds_bpermute.
//   * The four partial tiles are summed in wave order through LDS.
//
// Lane r + 16g of an operand fragment holds 16-byte chunks g and 4+g of its
// row's k-block (the k-assignment every path uses).  The product is taken
// as D = W * A^T: lane l holds output row m0 + 16i + l%16 and columns
// n0 + 16j + 4(l/16) .. +3, so one scale product per tile covers the lane's
// four elements and the store is one vector.
// ---------------------------------------------------------------------------
struct RawFragment {
  u32x4 lo, hi;
};

// Row-major operand: lane 4r+c reads chunks c and 4+c of row r.
AKAS_DEV RawFragment load_raw_fragment(const uint8_t* row_kblock, int chunk) {
  return {*reinterpret_cast<const u32x4*>(row_kblock + 16 * chunk),
          *reinterpret_cast<const u32x4*>(row_kblock + 64 + 16 * chunk)};
}

// lane r + 16g takes lane 4r + g
AKAS_DEV v8i to_mfma_order(const RawFragment& f, int sel) {
  v8i v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = __builtin_amdgcn_ds_bpermute(sel, (int)f.lo[e]);
    v[4 + e] = __builtin_amdgcn_ds_bpermute(sel, (int)f.hi[e]);
  }
  return v;
}

AKAS_DEV v8i as_fragment(const RawFragment& f) {
  v8i v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = (int)f.lo[e];
    v[4 + e] = (int)f.hi[e];
  }
  return v;
}

constexpr int kSplitQuarters = 4;  // k-split of a workgroup: four waves
constexpr int kBufferDword3 = 0x00020000;  // buffer resource word 3 (raw 32-bit data)
constexpr int kSplitKbw = 4;       // k-blocks per wave: 2048-deep partitions

// PF: activation k-blocks loaded up front (the rest follow the first
// multiplies).  AFIRST: activation loads ahead of the weight loads (small
// tiles, whose activations are quick to land) or right behind them (large
// tiles: the weights' HBM latency goes first).
//
// MH: waves per k-quarter (1 or 2).  With MH = 2 the workgroup has eight
// waves: wave (kq, mh) multiplies rows 16*MT*mh .. +16*MT-1 of the tile over
// quarter kq, the two waves of a quarter each stage half of its weight
// slice, and each SIMD holds two waves, so one wave's MFMAs overlap the
// other's loads and folds.
template <int MT, int NT, int PF, int AFIRST, int AF, int OUT, int SDT, int MH = 1>
__global__ __launch_bounds__(64 * kSplitQuarters * MH) void dense_split_kernel(DenseArgs p) {
  constexpr int KBW = kSplitKbw, BM = 16 * MT * MH, BN = 16 * NT;
  constexpr int WT = MT * NT;                        // output tiles per wave
  constexpr int WROW = KBW * kBlock;                 // bytes of a weight row per quarter
  constexpr int QUARTER = BN * WROW;                 // LDS bytes of one quarter's slice
  constexpr int RED = WT * kWave * 16;               // LDS bytes of one wave's partials
  static_assert(BN % (2 * MH) == 0 && WROW == 512, "two 512-byte weight rows per load");
  static_assert(MH * RED <= QUARTER, "a quarter's partials overwrite its weight slice");
  static_assert(PF >= 1 && PF <= KBW, "activation prefetch depth");
  constexpr int LDS_BYTES = kSplitQuarters * QUARTER;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];

  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = wave % kSplitQuarters, mh = wave / kSplitQuarters;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = p.N / BN;
  // m-tiles of one column block are adjacent, so both reads of a weight
  // slice land in the same XCD's L2
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int tm = id % tiles_m, tn = id / tiles_m;
  const int m0 = tm * BM + mh * 16 * MT, n0 = tn * BN;  // m0: this wave's first row
  const int KB = p.K / kBlock;
  const int part = blockIdx.y;
  const int kb0 = part * p.kb_per_part + kq * KBW;
  uint8_t* wq = lds + kq * QUARTER;  // this quarter's weight slice

  // Rows past M re-read the last row (or 16-row tile) and are never stored.
  uint32_t arow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) arow[i] = (uint32_t)min(m0 + 16 * i + r, p.M - 1);

  // Scales first (the k-block loop waits on loads in issue order).
  v4f sa[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) sa[i] = *reinterpret_cast<const v4f*>(p.as + (int64_t)arow[i] * KB + kb0);
  // Raw weight-scale bits: converting them here would wait for the loads
  // before the weight slice is even requested.
  uint32_t swraw[KBW][NT];
#pragma unroll
  for (int s = 0; s < KBW; ++s)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t at = (int64_t)((n0 + 16 * j) / kBlock) * KB + kb0 + s;
      if constexpr (SDT == AKAS_DTYPE_F32)
        swraw[s][j] = reinterpret_cast<const uint32_t*>(p.ws)[at];
      else
        swraw[s][j] = reinterpret_cast<const uint16_t*>(p.ws)[at];
    }

  // Activation k-blocks of this quarter.
  const int lr = lane >> 2, lc = lane & 3;
  const int sel = (4 * r + g) << 2;
  const int last_tile = (p.M - 1) >> 4;
  // Buffer loads: the tile offset of a fragment is wave-uniform (scalar),
  // so a load costs one vector register of address for the whole wave.
  const int a_bytes = AF ? ((p.M + 15) >> 4) * KB * 2048 : p.M * p.K;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.a), (short)0, a_bytes, kBufferDword3);
  auto load_a = [&](int i, int s) -> RawFragment {
    RawFragment f;
    if constexpr (AF) {
      const int t = ((min((m0 >> 4) + i, last_tile) * KB + kb0 + s) << 11);
      f.lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, 16 * lane, t, 0));
      f.hi = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, 16 * lane, t + 1024, 0));
    } else {
      const int row = min(m0 + 16 * i + lr, p.M - 1);
      const int off = row * p.K + (kb0 + s) * kBlock + 16 * lc;
      f.lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, 0, 0));
      f.hi = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off + 64, 0, 0));
    }
    return f;
  };
  RawFragment araw[PF][MT];
  auto issue_a = [&]() {
#pragma unroll
    for (int s = 0; s < PF; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) araw[s][i] = load_a(i, s);
  };

  // The wave's share of its quarter's weight slice (rows mh*BN/MH ..), two
  // rows of 512 contiguous bytes per load.
  constexpr int WLOADS = BN / 2 / MH;
  const int wl_row = lane >> 5, wl_chunk = lane & 31;
  const int wl_row0 = mh * (BN / MH);
  const uint8_t* wsrc = p.w + (int64_t)(n0 + wl_row0 + wl_row) * p.K + (int64_t)kb0 * kBlock + 16 * wl_chunk;
  u32x4 wl[WLOADS];
  auto issue_w = [&]() {
#pragma unroll
    for (int q = 0; q < WLOADS; ++q) wl[q] = *reinterpret_cast<const u32x4*>(wsrc + (int64_t)(2 * q) * p.K);
  };
  if constexpr (AFIRST) {
    issue_a();
    __builtin_amdgcn_sched_barrier(0);
    issue_w();
  } else {
    issue_w();
    __builtin_amdgcn_sched_barrier(0);
    issue_a();
  }
  __builtin_amdgcn_sched_barrier(0);

  // Weight slice into LDS: row rho, chunk c at rho*512 + 16*(c ^ (rho & 15)),
  // so the sixteen rows of a fragment read hit sixteen different banks.
#pragma unroll
  for (int q = 0; q < WLOADS; ++q) {
    const int rho = wl_row0 + 2 * q + wl_row;
    *reinterpret_cast<u32x4*>(wq + rho * WROW + 16 * (wl_chunk ^ (rho & 15))) = wl[q];
  }
  if constexpr (MH > 1) __syncthreads();  // the other half of the slice

  float sw[KBW][NT];
#pragma unroll
  for (int s = 0; s < KBW; ++s)
#pragma unroll
    for (int j = 0; j < NT; ++j)
      sw[s][j] = __uint_as_float(SDT == AKAS_DTYPE_F32 ? swraw[s][j] : swraw[s][j] << 16);

  v4f acc[MT][NT];
#pragma unroll
  for (int s = 0; s < KBW; ++s) {
    const int slot = s % PF;
    v8i af[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) af[i] = AF ? as_fragment(araw[slot][i]) : to_mfma_order(araw[slot][i], sel);
    if (s + PF < KBW) {
      // refill this slot once its fragments are taken (not hoisted, which
      // would hold every k-block in registers at once)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MT; ++i) araw[slot][i] = load_a(i, s + PF);
    }
    v8i wf[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const uint8_t* wr = wq + (16 * j + r) * WROW;
      RawFragment wfr;
      wfr.lo = *reinterpret_cast<const u32x4*>(wr + 16 * ((8 * s + g) ^ r));
      wfr.hi = *reinterpret_cast<const u32x4*>(wr + 16 * ((8 * s + 4 + g) ^ r));
      wf[j] = as_fragment(wfr);
    }
    // m-tile by m-tile, so only one m-tile's products wait for their scale fold
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const v4f d = mfma_e4m3(wf[j], af[i]);
        const float c = sa[i][s] * sw[s][j];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] = s == 0 ? d[e] * c : __builtin_fmaf(d[e], c, acc[i][j][e]);
      }
  }

  // Tile t = i*NT + j is summed and stored by wave t % 4, in wave order;
  // partials go through LDS over each wave's own (finished) weight slice.
  v4f* red = reinterpret_cast<v4f*>(lds) + mh * WT * kWave;
  auto slot = [&](int q, int t) { return q * (QUARTER / 16) + t * kWave + lane; };
  const int64_t obase = (int64_t)part * p.part_stride;
  if constexpr (MH > 1) __syncthreads();  // both waves of a quarter are done with its slice
  if constexpr (AF && MH == 1) {
    // Fragment-major activations, four waves: the owner keeps its own
    // partial in registers.  (With the batched form below, the compiler no
    // longer hoists both activation refills ahead of the first multiplies in
    // the 128-row four-wave instantiation: measured 13.2 -> 14.0 us per M=256
    // fp8_linear.  With eight waves the register-resident form spills.)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if ((i * NT + j) % kSplitQuarters != kq) red[slot(kq, i * NT + j)] = acc[i][j];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int t = i * NT + j;
        if (t % kSplitQuarters != kq) continue;
        v4f sum = kq == 0 ? acc[i][j] : red[slot(0, t)];
#pragma unroll
        for (int q = 1; q < kSplitQuarters; ++q) sum += q == kq ? acc[i][j] : red[slot(q, t)];
        const int row = m0 + 16 * i + r;
        if (row < p.M) store_out4<OUT>(p.out, obase + (int64_t)row * p.ldo + n0 + 16 * j + 4 * g, sum);
      }
  } else {
    // Row-major activations: every wave writes all of its partials, and the
    // owner issues every LDS read of its tiles before the first add (one
    // LDS round trip instead of three per tile; the tile index is runtime
    // here, so the owner's own partial comes back from LDS as well).
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) red[slot(kq, i * NT + j)] = acc[i][j];
    __syncthreads();
    constexpr int OWN = (WT + kSplitQuarters - 1) / kSplitQuarters;
    v4f parts[OWN][kSplitQuarters];
#pragma unroll
    for (int u = 0; u < OWN; ++u) {
      const int t = min(kSplitQuarters * u + kq, WT - 1);
#pragma unroll
      for (int q = 0; q < kSplitQuarters; ++q) parts[u][q] = red[slot(q, t)];
    }
#pragma unroll
    for (int u = 0; u < OWN; ++u) {
      const int t = kSplitQuarters * u + kq;
      if (t >= WT) break;
      v4f sum = parts[u][0];
#pragma unroll
      for (int q = 1; q < kSplitQuarters; ++q) sum += parts[u][q];
      const int i = t / NT, j = t % NT;
      const int row = m0 + 16 * i + r;
      if (row < p.M) store_out4<OUT>(p.out, obase + (int64_t)row * p.ldo + n0 + 16 * j + 4 * g, sum);
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill GEMM: 256x256 tiles streamed into LDS by the gfx950 copy engine
// (tile engine in gemm_dma.h).  N must be a multiple of 128 so that each
// wave's 128 output columns are either all inside the matrix or all outside;
// rows and columns past the ends are clamped on load and never stored.
// ---------------------------------------------------------------------------
template <int OUT, int SDT>
__global__ __launch_bounds__(dma::THREADS) void dense_dma_kernel(DenseArgs p) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (p.M + dma::BM - 1) / dma::BM, tiles_n = (p.N + dma::BN - 1) / dma::BN;
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  int tm, tn;
  grouped_tile(id, tiles_m, tiles_n, 8, tm, tn);
  const int m0 = tm * dma::BM, n0 = tn * dma::BN;
  const int KB = p.K / kBlock;
  const int part = blockIdx.y;
  const int kb0 = part * p.kb_per_part, kb1 = kb0 + p.kb_per_part;

  dma::AffinePlan plan;
  const bool copies_a = wave < 4;
  plan.src = copies_a ? p.a : p.w;
  plan.blk0 = wave * 8;
  {
    const int row = dma::piece_row(wave, 0, lane);
    plan.row0 = (uint32_t)((copies_a ? m0 : n0) + row);
    plan.lim = (uint32_t)((copies_a ? p.M : p.N) - 1);
    plan.ld = (uint32_t)p.K;
    plan.chunk = (uint32_t)dma::piece_chunk(row, lane);
  }
  plan.as = p.as;
  plan.soff = (uint32_t)min(m0 + (wave & 3) * 64 + lane, p.M - 1) * (uint32_t)KB;
  plan.scales = copies_a;
  // quarters of the last (partial) tiles that hold no row of A or of B
  plan.skip = (copies_a ? m0 : n0) + (wave & 3) * 64 >= (copies_a ? p.M : p.N);

  const int a_row0 = (wave & 3) * 64, b_row0 = (wave >> 2) * 128;
  const int col0 = n0 + b_row0;
  const bool live = m0 + a_row0 < p.M && col0 < p.N;  // wave-uniform
  // Weight scale of each k-block for this wave's 128-column block.  f32
  // scales are loaded per stage from global memory, so the first stage's
  // copies go out at once (a table in LDS first costs a load round trip per
  // tile: 2,011-2,046 against 2,041-2,068 TFLOP/s at M=8192, K=2048,
  // N=6144).  bf16 scales go through a float32 table in LDS over the
  // partition's k-blocks, because a bf16 load per stage made the compiler
  // spill in the main loop.
  dma::Acc acc;
  acc.clear();
  if constexpr (SDT == AKAS_DTYPE_F32) {
    const int64_t ws_base = (int64_t)min(col0 / kBlock, (p.N - 1) / kBlock) * KB;
    dma::run<false>(plan, acc, a_row0, b_row0, kb0, kb1, lane, [&](int kb) {
      const float w = load_scale_t<AKAS_DTYPE_F32>(p.ws, ws_base + kb);
      return float2{w, w};
    }, live);
  } else {
    const int nkb = kb1 - kb0;
    for (int i = tid; i < 2 * nkb; i += dma::THREADS) {
      const int h = i / nkb, k = kb0 + i % nkb;
      const int64_t at = (int64_t)min((n0 + 128 * h) / kBlock, (p.N - 1) / kBlock) * KB + k;
      dma::wtab[h][i % nkb] = load_scale_t<AKAS_DTYPE_BF16>(p.ws, at);
    }
    __syncthreads();
    const float* wrow = dma::wtab[wave >> 2];
    dma::run<false>(plan, acc, a_row0, b_row0, kb0, kb1, lane, [&](int kb) {
      const float w = wrow[kb - kb0];
      return float2{w, w};
    }, live);
  }
  const int rows = col0 < p.N ? min(64, p.M - (m0 + a_row0)) : 0;
  dma::store_tile_rows<OUT>(acc, p.out, wave, lane, rows,
                            (int64_t)part * p.part_stride + col0 + (int64_t)(m0 + a_row0) * p.ldo, p.ldo);
}

// ---------------------------------------------------------------------------
// Small-M MFMA GEMM: one 16-column tile per workgroup, four waves striding
// over the k-blocks with every operand fetched straight from global memory
// (weights stream once from HBM, activations hit L2), then a fixed-order
// LDS reduction of the four partial tiles.
// ---------------------------------------------------------------------------
template <int MT, int OUT, int SDT>
__global__ __launch_bounds__(256) void dense_small_kernel(DenseArgs p) {
  constexpr int U = MT <= 2 ? 4 : 2;  // k-blocks in flight per wave
  __shared__ __attribute__((aligned(16))) float red[4][MT][64][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int n0 = blockIdx.x * 16;
  const int part = blockIdx.y;
  const int KB = p.K / kBlock;
  const int kb0 = part * p.kb_per_part, kb1 = kb0 + p.kb_per_part;

  const uint8_t* wrow = p.w + (int64_t)(n0 + r16) * p.K + g * 32;
  const uint8_t* arow[MT];
  const float* srow[MT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int m = 16 * i + r16;
    arow[i] = m < p.M ? p.a + (int64_t)m * p.K + g * 32 : nullptr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int mo = 16 * i + 4 * g + e;
      srow[i][e] = mo < p.M ? p.as + (int64_t)mo * KB : nullptr;
    }
  }
  const int64_t ws_base = (int64_t)(n0 / kBlock) * KB;

  v4f acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int kb = kb0 + wave; kb < kb1; kb += 4 * U) {
    uint4 wl[U][2], al[U][MT][2];
    float sv[U][MT][4], wsv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kb + 4 * u;
      if (k < kb1) {
        const int64_t ko = (int64_t)k * kBlock;
        wl[u][0] = *reinterpret_cast<const uint4*>(wrow + ko);
        wl[u][1] = *reinterpret_cast<const uint4*>(wrow + ko + 16);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          if (arow[i]) {
            al[u][i][0] = *reinterpret_cast<const uint4*>(arow[i] + ko);
            al[u][i][1] = *reinterpret_cast<const uint4*>(arow[i] + ko + 16);
          } else {
            al[u][i][0] = al[u][i][1] = make_uint4(0, 0, 0, 0);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) sv[u][i][e] = srow[i][e] ? srow[i][e][k] : 0.f;
        }
        wsv[u] = load_scale_t<SDT>(p.ws, ws_base + k);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kb + 4 * u;
      if (k < kb1) {
        v8i bf;
        bf[0] = wl[u][0].x; bf[1] = wl[u][0].y; bf[2] = wl[u][0].z; bf[3] = wl[u][0].w;
        bf[4] = wl[u][1].x; bf[5] = wl[u][1].y; bf[6] = wl[u][1].z; bf[7] = wl[u][1].w;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          v8i af;
          af[0] = al[u][i][0].x; af[1] = al[u][i][0].y; af[2] = al[u][i][0].z; af[3] = al[u][i][0].w;
          af[4] = al[u][i][1].x; af[5] = al[u][i][1].y; af[6] = al[u][i][1].z; af[7] = al[u][i][1].w;
          const v4f pr = mfma_e4m3(af, bf);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[i][e] = __builtin_fmaf(pr[e], sv[u][i][e] * wsv[u], acc[i][e]);
        }
      }
    }
  }

#pragma unroll
  for (int i = 0; i < MT; ++i)
    *reinterpret_cast<float4*>(&red[wave][i][lane][0]) =
        make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
  __syncthreads();
  // wave w finalizes m-tiles w, w+4, ... ; fixed summation order 0..3
  const int64_t obase = (int64_t)part * p.part_stride;
  for (int i = wave; i < MT; i += 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = red[0][i][lane][e];
      v += red[1][i][lane][e];
      v += red[2][i][lane][e];
      v += red[3][i][lane][e];
      const int row = 16 * i + 4 * g + e, col = n0 + r16;
      if (row < p.M) store_out<OUT>(p.out, obase + (int64_t)row * p.ldo + col, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Wide small-M MFMA GEMM (M <= 64): one workgroup of NTW x KS waves covers
// 16*NTW columns and the partition's whole k range.  The activation slab
// (codes and scales of all its rows) is staged in LDS once per workgroup,
// every wave issues all of its weight loads up front (k-blocks strided by
// KS), multiplies, and the KS partial tiles are summed in a fixed order.
// Weights stream from HBM exactly once; activations are read from L2 once
// per workgroup instead of once per wave.
// ---------------------------------------------------------------------------
constexpr int kWideBatch = 2;  // k-blocks of weights in flight per wave

template <int MT, int NTW, int KS>
constexpr size_t wide_lds_bytes(int kbp) {
  const size_t stage = (size_t)kbp * 16 * MT * (128 + 4);
  const size_t red = (size_t)KS * NTW * MT * 64 * 16;
  if (MT == 1) return ((stage + 15) & ~(size_t)15) + red;  // partials beside the slab
  return stage > red ? stage : red;
}

//
// QX = 0: the slab is staged from prequantized codes and scales (a, as).
// QX = DT + 1: the slab is quantized from the f32/f16/bf16 activations x
// while it is staged -- 16 lanes per 1x128 group, the same quantize8 as the
// standalone quantizer, so the codes are identical -- which saves the
// quantizer's launch and its codes' round trip for decode-sized batches.
//
// CW: output columns per workgroup (NTW 16-column tiles; the last tile may
// hold fewer than 16 valid columns -- its other lanes re-read the last valid
// weight row and store nothing), so that N / CW workgroups can match the CU
// count: at N = 6144, 24 columns give 256 workgroups where 32 give 192.
// A 24-column workgroup loads its weight scales per lane (its tiles can
// straddle a 128-column scale block).
template <int MT, int NTW, int KS, int OUT, int SDT, int QX = 0, int CW = 16 * NTW>
__global__ __launch_bounds__(64 * NTW * KS) void dense_wide_kernel(DenseArgs p) {
  static_assert(CW > 16 * (NTW - 1) && CW <= 16 * NTW, "columns per workgroup fill NTW tiles");
  constexpr int THREADS = 64 * NTW * KS;
  constexpr int ROWS = 16 * MT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int KB = p.K / kBlock;
  const int part = blockIdx.y;
  const int kb0 = part * p.kb_per_part, kbp = p.kb_per_part;
  uint8_t* lds_a = smem;                                            // [kbp][ROWS][128]
  float* lds_s = reinterpret_cast<float*>(smem + (size_t)kbp * ROWS * 128);  // [kbp][ROWS]
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = wave % NTW, ks = wave / NTW;
  const int n0 = blockIdx.x * CW + nt * 16;
  const int valid = min(16, CW - nt * 16);  // valid columns of this tile
  const int g = lane >> 4, r16 = lane & 15;
  const int col = n0 + min(r16, valid - 1);  // this lane's weight row
  const uint8_t* wrow = p.w + (int64_t)col * p.K + g * 32;
  // Only a tile that is not 16-column aligned (CW = 24) can straddle a
  // 128-column scale block; the others keep a wave-uniform (scalar) scale.
  const int64_t ws_base = (int64_t)((CW % 16 ? col : n0) / kBlock) * KB;

  // 1. first batch of this wave's weight loads (local k-blocks ks, ks+KS, ...)
  u32x4 wl[kWideBatch][2];
  float wsv[kWideBatch];
  auto issue = [&](int b) {
#pragma unroll
    for (int j = 0; j < kWideBatch; ++j) {
      // unconditional: a k-block past the partition re-reads its last one
      // (never multiplied), so the compiler can wait for each load alone
      const int lk = min(ks + KS * (b * kWideBatch + j), kbp - 1);
      const int64_t ko = (int64_t)(kb0 + lk) * kBlock;
      wl[j][0] = *reinterpret_cast<const u32x4*>(wrow + ko);
      wl[j][1] = *reinterpret_cast<const u32x4*>(wrow + ko + 16);
      wsv[j] = load_scale_t<SDT>(p.ws, ws_base + kb0 + lk);
    }
  };
  // Fused quantize: the first pass of activation loads goes out before the
  // weights, so quantizing waits only for them (loads complete in issue order).
  constexpr int GPP = THREADS / 16, PASS = 4;
  const int l16 = lane & 15, groups = QX ? p.M * kbp : 0;
  Raw8 xraw[PASS];
  if constexpr (QX != 0) {
#pragma unroll
    for (int u = 0; u < PASS; ++u) {
      // unconditional (clamped) so the compiler can wait for each load alone
      const int c = min((tid >> 4) + u * GPP, groups - 1);
      xraw[u] = load8_raw<QX - 1>(p.x, (int64_t)(c / kbp) * p.K + (int64_t)(kb0 + c % kbp) * kBlock + l16 * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  issue(0);
  __builtin_amdgcn_sched_barrier(0);

  // 2. stage the activation slab (rows past M are zero) and its scales
  if constexpr (QX == 0) {
    for (int c = tid; c < ROWS * kbp * 8; c += THREADS) {
      const int row = c / (kbp * 8), rem = c % (kbp * 8), lk = rem >> 3, ch = rem & 7;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row < p.M)
        v = *reinterpret_cast<const u32x4*>(p.a + (int64_t)row * p.K + (int64_t)(kb0 + lk) * kBlock + ch * 16);
      *reinterpret_cast<u32x4*>(lds_a + (size_t)lk * ROWS * 128 + lds_off(row, ch)) = v;
    }
    for (int c = tid; c < ROWS * kbp; c += THREADS) {
      const int lk = c / ROWS, row = c % ROWS;
      lds_s[c] = row < p.M ? p.as[(int64_t)row * KB + kb0 + lk] : 0.f;
    }
  } else {
    // rows past M: zero codes and scales, no loads
    for (int c = p.M * kbp * 8 + tid; c < ROWS * kbp * 8; c += THREADS) {
      const int row = c / (kbp * 8), rem = c % (kbp * 8), lk = rem >> 3, ch = rem & 7;
      *reinterpret_cast<u32x4*>(lds_a + (size_t)lk * ROWS * 128 + lds_off(row, ch)) = u32x4{0u, 0u, 0u, 0u};
    }
    for (int c = tid; c < ROWS * kbp; c += THREADS)
      if (c % ROWS >= p.M) lds_s[c] = 0.f;
    // live groups (row, lk), one per 16 lanes, PASS groups per lane block with
    // all their loads issued before any is used; lane l16 holds values
    // 8*l16 .. 8*l16+7, i.e. half (l16 & 1) of chunk l16 / 2
    for (int c0 = tid >> 4; c0 < groups; c0 += PASS * GPP) {
      float v[PASS][8];
      const bool first = c0 == (tid >> 4);
#pragma unroll
      for (int u = 0; u < PASS; ++u) {
        const int c = c0 + u * GPP;
        if (c < groups) {
          if (first)
            unpack8<QX - 1>(xraw[u], v[u]);
          else
            load8<QX - 1>(p.x, (int64_t)(c / kbp) * p.K + (int64_t)(kb0 + c % kbp) * kBlock + l16 * 8, v[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < PASS; ++u) {
        const int c = c0 + u * GPP;
        if (c < groups) {  // uniform across the group's 16 lanes
          const int row = c / kbp, lk = c % kbp;
          float sc;
          const uint2 codes = quantize8(v[u], sc);
          *reinterpret_cast<uint2*>(lds_a + (size_t)lk * ROWS * 128 + lds_off(row, l16 >> 1) + (l16 & 1) * 8) = codes;
          if (l16 == 0) lds_s[lk * ROWS + row] = sc;
        }
      }
    }
  }
  __syncthreads();

  // 3. multiply batch by batch
  v4f acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
  const int batches = (kbp + KS * kWideBatch - 1) / (KS * kWideBatch);
  for (int b = 0; b < batches; ++b) {
    if (b > 0) issue(b);
#pragma unroll
    for (int j = 0; j < kWideBatch; ++j) {
      const int lk = ks + KS * (b * kWideBatch + j);
      if (lk < kbp) {
        v8i bf;
        bf[0] = wl[j][0][0]; bf[1] = wl[j][0][1]; bf[2] = wl[j][0][2]; bf[3] = wl[j][0][3];
        bf[4] = wl[j][1][0]; bf[5] = wl[j][1][1]; bf[6] = wl[j][1][2]; bf[7] = wl[j][1][3];
        const uint8_t* at = lds_a + (size_t)lk * ROWS * 128;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const v8i af = lds_fragment(at, 16 * i, lane);
          const float4 s4 = *reinterpret_cast<const float4*>(lds_s + lk * ROWS + 16 * i + 4 * g);
          const v4f pr = mfma_e4m3(af, bf);
          acc[i][0] = __builtin_fmaf(pr[0], s4.x * wsv[j], acc[i][0]);
          acc[i][1] = __builtin_fmaf(pr[1], s4.y * wsv[j], acc[i][1]);
          acc[i][2] = __builtin_fmaf(pr[2], s4.z * wsv[j], acc[i][2]);
          acc[i][3] = __builtin_fmaf(pr[3], s4.w * wsv[j], acc[i][3]);
        }
      }
    }
  }

  // 4. fixed-order sum of the KS partial tiles (LDS slab reused when the
  // partials do not fit beside it)
  float* red;
  if constexpr (MT == 1) {
    red = reinterpret_cast<float*>(smem + (((size_t)kbp * 16 * MT * (128 + 4) + 15) & ~(size_t)15));
  } else {
    __syncthreads();
    red = reinterpret_cast<float*>(smem);
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
    *reinterpret_cast<float4*>(red + (((ks * NTW + nt) * MT + i) * 64 + lane) * 4) =
        make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
  __syncthreads();
  if (ks == 0) {
    const int64_t obase = (int64_t)part * p.part_stride;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = red[((nt * MT + i) * 64 + lane) * 4 + e];
        for (int q = 1; q < KS; ++q) v += red[(((q * NTW + nt) * MT + i) * 64 + lane) * 4 + e];
        const int row = 16 * i + 4 * g + e;
        if (row < p.M && r16 < valid) store_out<OUT>(p.out, obase + (int64_t)row * p.ldo + n0 + r16, v);
      }
  }
}

// Serial f32 sum over partitions (src/akas/ops/linear/cuda.py:1369-1402).
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ partial,
                                                    void* __restrict__ out, int out_dtype,
                                                    int64_t rows, int64_t o, int parts) {
  const int64_t n = rows * o;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / o, col = i % o;
    const float* src = partial + row * parts * o + col;
    float t = 0.f;
    for (int q = 0; q < parts; ++q) t += src[(int64_t)q * o];
    store_elem(out, i, t, out_dtype);
  }
}

template <int BM, int BN, int WMW, int WNW, int DEPTH, int OUT, int SDT>
static void launch_tiled(const DenseArgs& a, int parts, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  dense_tiled_kernel<BM, BN, WMW, WNW, DEPTH, OUT, SDT>
      <<<dim3(tiles, parts), 64 * WMW * WNW, 0, s>>>(a);
}

// The DMA-fed 256x256 kernel takes over once its tiles cover the GPU at
// least about once (fewer, larger tiles idle too many CUs) and the output
// rows are 16-byte aligned for its vector stores.
static bool dma_fits(const DenseArgs& a, int parts) {
  const int esz = a.out_dtype == AKAS_DTYPE_F32 ? 4 : 2;
  const int64_t tiles = (int64_t)((a.M + dma::BM - 1) / dma::BM) * ((a.N + dma::BN - 1) / dma::BN);
  return a.N % 128 == 0 && tiles * parts >= 240 && a.kb_per_part <= dma::MAX_KB && (a.ldo * esz) % 16 == 0 &&
         (a.part_stride * esz) % 16 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0;
}

// The split kernel: 2048-deep partitions, N a multiple of its 48-column
// tiles, aligned 4-element output vectors and activation-scale vectors,
// 32-bit code offsets.
constexpr int kSplitNt = 3;
// Column tile of the split kernel: 48 columns where N allows, else narrower
// tiles for the other multiples of 16, so that small N still spreads over
// many workgroups (16 columns below 2048 columns, else 32).
static int split_nt(const DenseArgs& a) {
  if (a.N % (16 * kSplitNt) == 0) return kSplitNt;
  if (a.N % 32 == 0 && a.N >= 2048) return 2;
  return a.N % 16 == 0 ? 1 : 0;
}

static bool split_fits(const DenseArgs& a) {
  const int esz = a.out_dtype == AKAS_DTYPE_F32 ? 4 : 2;
  // 32-bit buffer offsets: the fragment-major codes hold M rounded up to 16 rows
  return a.kb_per_part == kSplitQuarters * kSplitKbw && split_nt(a) > 0 &&
         (int64_t)((a.M + 15) & ~15) * a.K < (1ll << 31) && (a.K / kBlock) % 4 == 0 && a.ldo % 4 == 0 &&
         a.part_stride % 4 == 0 && reinterpret_cast<uintptr_t>(a.out) % (4 * esz) == 0 &&
         reinterpret_cast<uintptr_t>(a.as) % 16 == 0;
}

static bool split_applies(const DenseArgs& a, int parts) {
  return a.M > 16 && a.M <= 256 && split_fits(a) && parts >= 1;
}

template <int MT, int PF, int AFIRST, int AF, int OUT, int SDT, int MH = 1, int NT = kSplitNt>
static void launch_split(const DenseArgs& a, int parts, hipStream_t s) {
  const int tiles = ((a.M + 16 * MT * MH - 1) / (16 * MT * MH)) * (a.N / (16 * NT));
  dense_split_kernel<MT, NT, PF, AFIRST, AF, OUT, SDT, MH>
      <<<dim3(tiles, parts), 64 * kSplitQuarters * MH, 0, s>>>(a);
}

// One row-tile configuration with the column tile split_nt() picks.
template <int MT, int PF, int AFIRST, int AF, int OUT, int SDT, int MH>
static void launch_split_nt(const DenseArgs& a, int parts, hipStream_t s) {
  switch (split_nt(a)) {
    case 1: launch_split<MT, PF, AFIRST, AF, OUT, SDT, MH, 1>(a, parts, s); break;
    case 2: launch_split<MT, PF, AFIRST, AF, OUT, SDT, MH, 2>(a, parts, s); break;
    default: launch_split<MT, PF, AFIRST, AF, OUT, SDT, MH>(a, parts, s);
  }
}

// Row tiles of the split kernel by M (16 < M <= 256), two tiles per column
// block so that the grid covers 256 CUs at N = 6144.  Above 64 rows the
// tile runs on eight waves (two row halves per k-quarter): M=256 GEMM 11.9
// -> 10.8 us and fp8_linear 13.2 -> 12.7 us, M=128 fp8_linear 10.2 -> 9.8 us
// against four waves; at 64 rows and below eight waves were slower.
template <int AF, int OUT, int SDT>
static void launch_split_m(const DenseArgs& a, int parts, hipStream_t s) {
  if (a.M <= 32)
    launch_split_nt<1, 4, 1, AF, OUT, SDT, 1>(a, parts, s);
  else if (a.M <= 64)
    launch_split_nt<2, 4, 1, AF, OUT, SDT, 1>(a, parts, s);
  else if (a.M <= 128)
    launch_split_nt<2, 2, 0, AF, OUT, SDT, 2>(a, parts, s);
  else
    launch_split_nt<4, 2, 0, AF, OUT, SDT, 2>(a, parts, s);
}

template <int OUT, int SDT>
static void launch_dma(const DenseArgs& a, int parts, hipStream_t s) {
  const int tiles = ((a.M + dma::BM - 1) / dma::BM) * ((a.N + dma::BN - 1) / dma::BN);
  dense_dma_kernel<OUT, SDT><<<dim3(tiles, parts), dma::THREADS, 0, s>>>(a);
}

// The direct-load small-M kernel (up to 64 rows) by its row count.
template <int OUT, int SDT>
static void launch_small(const DenseArgs& a, int parts, hipStream_t s) {
  if (a.M <= 16)
    dense_small_kernel<1, OUT, SDT><<<dim3(a.N / 16, parts), 256, 0, s>>>(a);
  else if (a.M <= 32)
    dense_small_kernel<2, OUT, SDT><<<dim3(a.N / 16, parts), 256, 0, s>>>(a);
  else
    dense_small_kernel<4, OUT, SDT><<<dim3(a.N / 16, parts), 256, 0, s>>>(a);
}

// Returns false (the caller takes another kernel) when the tile does not
// fit or the kernel's dynamic LDS limit cannot be raised on this device.
template <int MT, int NTW, int KS, int OUT, int SDT, int QX = 0, int CW = 16 * NTW>
static bool launch_wide(const DenseArgs& a, int parts, hipStream_t s) {
  const size_t lds = wide_lds_bytes<MT, NTW, KS>(a.kb_per_part);
  if (lds > 160 * 1024 || a.N % CW) return false;
  auto kern = dense_wide_kernel<MT, NTW, KS, OUT, SDT, QX, CW>;
  // The 160 KB dynamic LDS limit, raised once per device for this kernel
  // (bit d: done on device d).
  static std::atomic<uint64_t> configured{0};
  const int dev = current_device();
  if (dev < 0) return false;
  if (!((configured.load(std::memory_order_acquire) >> dev) & 1u)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) {
      // The caller launches another kernel instead; the failed call must not
      // leave its error for the launch check after that kernel.
      (void)hipGetLastError();
      return false;
    }
    configured.fetch_or(uint64_t{1} << dev, std::memory_order_release);
  }
  kern<<<dim3(a.N / CW, parts), 64 * NTW * KS, lds, s>>>(a);
  return true;
}

// Columns per workgroup of the M <= 16 wide kernel: the widest of 32, 24,
// 16 and 8 that gives at least about one workgroup per CU over the grid
// (weights are the bytes that matter there, and a CU's outstanding misses
// bound its share), else the narrowest that divides N.
static int wide_columns(int n, int parts) {
  const int cus = device_cus();
  for (int cw : {32, 24, 16, 8})
    if (n % cw == 0 && (int64_t)(n / cw) * parts >= cus - cus / 16) return cw;
  for (int cw : {8, 16, 24, 32})
    if (n % cw == 0) return cw;
  return 32;
}

// The M <= 16 wide kernel (MT = 1) at the column count wide_columns picks.
template <int OUT, int SDT, int QX = 0>
static bool launch_wide_m16(const DenseArgs& a, int parts, hipStream_t s) {
  switch (wide_columns(a.N, parts)) {
    case 24: return launch_wide<1, 2, 8, OUT, SDT, QX, 24>(a, parts, s);
    case 16: return launch_wide<1, 1, 8, OUT, SDT, QX, 16>(a, parts, s);
    case 8: return launch_wide<1, 1, 8, OUT, SDT, QX, 8>(a, parts, s);
    default: return launch_wide<1, 2, 8, OUT, SDT, QX>(a, parts, s);
  }
}

// Kernel choice by shape, in order:
//   16 < M <= 256 with 2048-deep partitions   the split kernel
//   M <= 64                                   the wide kernel (activations
//                                             staged once per workgroup in LDS),
//                                             else the direct small kernel
//   M > 256 whose 256x256 tiles fill the GPU  the DMA-fed prefill kernel
//   otherwise                                 64x64 tiles up to 256 rows, then
//                                             256x128 tiles when they fill the
//                                             GPU, else 128x128
// Tiled kernels need N to be a multiple of BN (affine B rows); shapes that
// fit none of these fall back to 64-row slices of the direct small kernel.
template <int OUT, int SDT>
static void launch_dense_t(const DenseArgs& a, int parts, hipStream_t s) {
  bool done = false;
  if (split_applies(a, parts)) {
    launch_split_m<0, OUT, SDT>(a, parts, s);
    return;
  }
  if (a.M <= 16)
    done = launch_wide_m16<OUT, SDT>(a, parts, s);
  else if (a.M <= 32)
    done = launch_wide<2, 2, 8, OUT, SDT>(a, parts, s);
  else if (a.M <= 64)
    done = launch_wide<4, 2, 8, OUT, SDT>(a, parts, s);
  if (done) return;
  if (a.M <= 64) {
    launch_small<OUT, SDT>(a, parts, s);
  } else if (a.M > 256 && dma_fits(a, parts)) {
    launch_dma<OUT, SDT>(a, parts, s);
  } else if (a.M <= 256 && a.N % 64 == 0) {
    launch_tiled<64, 64, 2, 2, 2, OUT, SDT>(a, parts, s);
  } else if (a.N % 128 == 0 && (int64_t)((a.M + 255) / 256) * (a.N / 128) >= 512) {
    launch_tiled<256, 128, 4, 2, 1, OUT, SDT>(a, parts, s);
  } else if (a.N % 128 == 0) {
    launch_tiled<128, 128, 2, 2, 1, OUT, SDT>(a, parts, s);
  } else {
    const int esz = OUT == AKAS_DTYPE_F32 ? 4 : 2;
    for (int m0 = 0; m0 < a.M; m0 += 64) {
      DenseArgs b = a;
      b.M = min(64, a.M - m0);
      b.a = a.a + (int64_t)m0 * a.K;
      b.as = a.as + (int64_t)m0 * (a.K / kBlock);
      b.out = reinterpret_cast<char*>(a.out) + (int64_t)m0 * a.ldo * esz;
      launch_small<OUT, SDT>(b, parts, s);
    }
  }
}

template <int OUT>
static void launch_dense_o(const DenseArgs& a, int parts, hipStream_t s) {
  if (a.ws_dtype == AKAS_DTYPE_F32)
    launch_dense_t<OUT, AKAS_DTYPE_F32>(a, parts, s);
  else
    launch_dense_t<OUT, AKAS_DTYPE_BF16>(a, parts, s);
}

// fp8_linear's split-kernel path: activations quantized fragment-major.
template <int OUT>
static void launch_split_frag_o(const DenseArgs& a, hipStream_t s) {
  if (a.ws_dtype == AKAS_DTYPE_F32)
    launch_split_m<1, OUT, AKAS_DTYPE_F32>(a, 1, s);
  else
    launch_split_m<1, OUT, AKAS_DTYPE_BF16>(a, 1, s);
}

static int launch_split_frag(const DenseArgs& a, hipStream_t s) {
  switch (a.out_dtype) {
    case AKAS_DTYPE_F32: launch_split_frag_o<AKAS_DTYPE_F32>(a, s); break;
    case AKAS_DTYPE_BF16: launch_split_frag_o<AKAS_DTYPE_BF16>(a, s); break;
    default: launch_split_frag_o<AKAS_DTYPE_F16>(a, s);
  }
  return hipGetLastError() == hipSuccess ? AKAS_OK : AKAS_ERR_LAUNCH;
}

int launch_dense(const DenseArgs& a, int parts, hipStream_t s) {
  switch (a.out_dtype) {
    case AKAS_DTYPE_F32: launch_dense_o<AKAS_DTYPE_F32>(a, parts, s); break;
    case AKAS_DTYPE_BF16: launch_dense_o<AKAS_DTYPE_BF16>(a, parts, s); break;
    default: launch_dense_o<AKAS_DTYPE_F16>(a, parts, s);
  }
  return hipGetLastError() == hipSuccess ? AKAS_OK : AKAS_ERR_LAUNCH;
}

// Decode-sized fp8_linear in one launch: the wide kernel quantizes x while
// staging it.  False when the shape does not fit the wide kernel.
// Up to kFusedQuantizeRows rows (the wide kernel's one-tile slab): the x
// loads go out ahead of the weights, so quantizing overlaps the weight
// stream, and the launch saved outweighs every workgroup re-quantizing the
// slab (K=2048, N=6144: fused 5.1 / 6.0 / 7.7 us vs 7.5 / 7.9 / 8.3 us
// quantize + GEMM at M=1 / 4 / 16).  Larger batches use the split kernel.
constexpr int kFusedQuantizeRows = 16;

template <int OUT, int SDT, int QX>
static bool launch_fused_small_t(const DenseArgs& a, hipStream_t s) {
  // Every workgroup quantizes the whole slab, so above 8 rows the extra
  // workgroups of narrower tiles cost more than their smaller weight share
  // saves (M=16, N=6144: 7.26 us at 32 columns, 7.37 us at 24).
  if (a.M <= 8) return launch_wide_m16<OUT, SDT, QX>(a, 1, s);
  if (a.M <= 16) return launch_wide<1, 2, 8, OUT, SDT, QX>(a, 1, s);
  return false;
}

template <int OUT, int SDT>
static bool launch_fused_small_o(const DenseArgs& a, hipStream_t s) {
  switch (a.x_dtype) {
    case AKAS_DTYPE_F32: return launch_fused_small_t<OUT, SDT, AKAS_DTYPE_F32 + 1>(a, s);
    case AKAS_DTYPE_F16: return launch_fused_small_t<OUT, SDT, AKAS_DTYPE_F16 + 1>(a, s);
    default: return launch_fused_small_t<OUT, SDT, AKAS_DTYPE_BF16 + 1>(a, s);
  }
}

template <int OUT>
static bool launch_fused_small_s(const DenseArgs& a, hipStream_t s) {
  return a.ws_dtype == AKAS_DTYPE_F32 ? launch_fused_small_o<OUT, AKAS_DTYPE_F32>(a, s)
                                      : launch_fused_small_o<OUT, AKAS_DTYPE_BF16>(a, s);
}

static bool launch_fused_small(const DenseArgs& a, hipStream_t s) {
  switch (a.out_dtype) {
    case AKAS_DTYPE_F32: return launch_fused_small_s<AKAS_DTYPE_F32>(a, s);
    case AKAS_DTYPE_BF16: return launch_fused_small_s<AKAS_DTYPE_BF16>(a, s);
    default: return launch_fused_small_s<AKAS_DTYPE_F16>(a, s);
  }
}

static inline bool float_dtype(int d) {
  return d == AKAS_DTYPE_F32 || d == AKAS_DTYPE_F16 || d == AKAS_DTYPE_BF16;
}
static inline bool scale_dtype_ok(int d) { return d == AKAS_DTYPE_F32 || d == AKAS_DTYPE_BF16; }
static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace akas

using namespace akas;

// Deep products at decode-sized batches: 2048-deep partitions of the split
// kernel with f32 partials, then the serial merge.  0 when not taken.
constexpr int kSplitDepth = kSplitQuarters * kSplitKbw * kBlock;  // 2048
static int linear_partitions(int64_t r, int64_t k) {
  if (r <= kFusedQuantizeRows || r > 256 || k <= kSplitDepth || k % kSplitDepth) return 0;
  return (int)(k / kSplitDepth);
}

extern "C" size_t akas_fp8_linear_workspace_size(int64_t r, int64_t k, int64_t o) {
  if (r <= 0 || k <= 0) return 0;
  // codes: rows rounded up to the 16-row tiles of the fragment-major layout
  size_t n = align256((size_t)((r + 15) & ~15ll) * k) + align256((size_t)r * (k / kBlock) * sizeof(float));
  const int parts = linear_partitions(r, k);
  if (parts > 0 && o > 0) n += (size_t)r * parts * o * sizeof(float);  // f32 partials
  return n;
}

// Host checks of fp8_linear's arguments, before any workspace is looked at.
static int check_linear(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                        int scale_dtype, void* out, int out_dtype, int64_t r, int64_t k,
                        int64_t o) {
  if (r < 0 || k <= 0 || o <= 0 || k % kBlock || o % 16 || r > 0x7FFFFFFF || o > 0x7FFFFFFF ||
      k > 0x7FFFFFFF)
    return AKAS_ERR_GEOMETRY;
  if (!float_dtype(x_dtype) || !float_dtype(out_dtype) || !scale_dtype_ok(scale_dtype))
    return AKAS_ERR_DTYPE;
  if ((uint64_t)r * k >= (1ull << 32) || (uint64_t)o * k >= (1ull << 32)) return AKAS_ERR_GEOMETRY;
  if (r == 0) return AKAS_OK;
  if (!x || !w || !w_scales || !out) return AKAS_ERR_NULL;
  return AKAS_OK;
}

// fp8_linear on validated arguments (r > 0) with a workspace of at least
// akas_fp8_linear_workspace_size(r, k, o) bytes.  What the workspace held
// before the call never reaches the output: the only workspace bytes read
// that the call did not write are the padding rows of the last 16-row
// activation tile, whose products land in output rows past r, which are
// never stored.  So the workspace needs no clearing between calls.
static int run_fp8_linear(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                          int scale_dtype, void* out, int out_dtype, void* workspace, int64_t r,
                          int64_t k, int64_t o, hipStream_t s) {
  if (r <= kFusedQuantizeRows) {
    DenseArgs f{nullptr, nullptr, w, w_scales, out, o, 0, (int)r, (int)o, (int)k,
                (int)(k / kBlock), scale_dtype, out_dtype, x, x_dtype};
    if (launch_fused_small(f, s))
      return hipGetLastError() == hipSuccess ? AKAS_OK : AKAS_ERR_LAUNCH;
  }
  uint8_t* codes = reinterpret_cast<uint8_t*>(workspace);
  float* scales = reinterpret_cast<float*>(codes + align256((size_t)((r + 15) & ~15ll) * k));
  const int parts = linear_partitions(r, k);
  if (parts > 0) {
    float* partial = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(scales) +
                                              align256((size_t)r * (k / kBlock) * sizeof(float)));
    DenseArgs p{codes, scales, w, w_scales, partial, (int64_t)parts * o, o, (int)r, (int)o,
                (int)k, (int)(k / kBlock / parts), scale_dtype, AKAS_DTYPE_F32, nullptr, 0};
    if (split_applies(p, parts)) {
      const int st = launch_quantize(x, x_dtype, codes, scales, r, k, true, s);
      if (st != AKAS_OK) return st;
      if (scale_dtype == AKAS_DTYPE_F32)
        launch_split_m<1, AKAS_DTYPE_F32, AKAS_DTYPE_F32>(p, parts, s);
      else
        launch_split_m<1, AKAS_DTYPE_F32, AKAS_DTYPE_BF16>(p, parts, s);
      const int64_t n = r * o, want = (n + 255) / 256;
      merge_kernel<<<(int)(want < 16384 ? want : 16384), 256, 0, s>>>(partial, out, out_dtype, r, o,
                                                                       parts);
      return hipGetLastError() == hipSuccess ? AKAS_OK : AKAS_ERR_LAUNCH;
    }
  }
  DenseArgs a{codes, scales, w, w_scales, out, o, 0, (int)r, (int)o, (int)k,
              (int)(k / kBlock), scale_dtype, out_dtype, nullptr, 0};
  const bool frag = split_applies(a, 1);
  const int st = launch_quantize(x, x_dtype, codes, scales, r, k, frag, s);
  if (st != AKAS_OK) return st;
  return frag ? launch_split_frag(a, s) : launch_dense(a, 1, s);
}

extern "C" int akas_fp8_linear(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                               int scale_dtype, void* out, int out_dtype, void* workspace,
                               size_t workspace_bytes, int64_t r, int64_t k, int64_t o,
                               void* stream) {
  const int st = check_linear(x, x_dtype, w, w_scales, scale_dtype, out, out_dtype, r, k, o);
  if (st != AKAS_OK || r == 0) return st;
  if (!workspace || workspace_bytes < akas_fp8_linear_workspace_size(r, k, o))
    return AKAS_ERR_WORKSPACE;
  return run_fp8_linear(x, x_dtype, w, w_scales, scale_dtype, out, out_dtype, workspace, r, k, o,
                        reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// fp8_linear without allocation: the workspace is `scratch`, a file-scope
// device array of AKAS_NOALLOC_SCRATCH_BYTES.  Every GPU the library runs on
// holds its own copy until the process ends.  Host code never passes the
// array's name to a kernel (on the host it names a stand-in, not device
// memory): the device address comes from hipGetSymbolAddress, taken once per
// device with that device current, and cached per device.  All calls on one
// GPU share its array, so calls that overlap in time on one GPU (different
// streams, or different host threads) race on it; calls ordered on one
// stream do not.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[AKAS_NOALLOC_SCRATCH_BYTES];

static std::atomic<void*> scratch_address[kMaxDevices];
static std::mutex scratch_mutex;

// Device address of the current device's `scratch`, or null when the device
// index is out of range or the runtime cannot resolve the symbol.
static void* current_scratch() {
  const int dev = current_device();
  if (dev < 0) return nullptr;
  void* p = scratch_address[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  p = scratch_address[dev].load(std::memory_order_relaxed);
  if (!p) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
    scratch_address[dev].store(q, std::memory_order_release);
    p = q;
  }
  return p;
}

extern "C" int akas_fp8_linear_noalloc(const void* x, int x_dtype, const uint8_t* w,
                                       const void* w_scales, int scale_dtype, void* out,
                                       int out_dtype, int64_t r, int64_t k, int64_t o,
                                       void* stream) {
  const int st = check_linear(x, x_dtype, w, w_scales, scale_dtype, out, out_dtype, r, k, o);
  if (st != AKAS_OK || r == 0) return st;
  if (akas_fp8_linear_workspace_size(r, k, o) > AKAS_NOALLOC_SCRATCH_BYTES)
    return AKAS_ERR_SCRATCH;
  void* ws = current_scratch();
  if (!ws) return AKAS_ERR_LAUNCH;
  return run_fp8_linear(x, x_dtype, w, w_scales, scale_dtype, out, out_dtype, ws, r, k, o,
                        reinterpret_cast<hipStream_t>(stream));
}

extern "C" int akas_projection_partial(const uint8_t* x, const float* activation_scales,
                                       const uint8_t* w, const void* w_scales, int scale_dtype,
                                       void* out, int out_dtype, int64_t r, int64_t k, int64_t o,
                                       int partitions, void* stream) {
  if (r < 0 || k <= 0 || o <= 0 || k % kBlock || o % 16 || partitions < 1 ||
      (k / kBlock) % partitions || r > 0x7FFFFFFF || o > 0x7FFFFFFF || k > 0x7FFFFFFF)
    return AKAS_ERR_GEOMETRY;
  if (!float_dtype(out_dtype) || !scale_dtype_ok(scale_dtype)) return AKAS_ERR_DTYPE;
  if (partitions > 1 && out_dtype != AKAS_DTYPE_F32) return AKAS_ERR_DTYPE;
  if ((uint64_t)r * k >= (1ull << 32) || (uint64_t)o * k >= (1ull << 32)) return AKAS_ERR_GEOMETRY;
  if (r == 0) return AKAS_OK;
  if (!x || !activation_scales || !w || !w_scales || !out) return AKAS_ERR_NULL;
  DenseArgs a{x, activation_scales, w, w_scales, out,
              partitions > 1 ? (int64_t)partitions * o : o, partitions > 1 ? o : 0,
              (int)r, (int)o, (int)k, (int)(k / kBlock / partitions), scale_dtype, out_dtype};
  return launch_dense(a, partitions, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int akas_projection_merge(const float* partial, void* out, int out_dtype, int64_t rows,
                                     int64_t o, int partitions, void* stream) {
  if (rows < 0 || o <= 0 || partitions < 1) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(out_dtype)) return AKAS_ERR_DTYPE;
  if (rows == 0) return AKAS_OK;
  if (!partial || !out) return AKAS_ERR_NULL;
  const int64_t n = rows * o;
  const int64_t want = (n + 255) / 256;
  const int grid = (int)(want < 16384 ? want : 16384);
  merge_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(partial, out, out_dtype,
                                                                        rows, o, partitions);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}
