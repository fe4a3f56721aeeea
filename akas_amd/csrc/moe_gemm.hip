// Grouped (per-expert) block-scaled FP8 GEMMs for gfx950:
//   expert_partial       -- gathered rows x expert weights, scattered to (row, rank)
//   fp8_expert_swiglu    -- gate and up products in one tile, SwiGLU, and
//                           per-128-column FP8 re-quantization in the epilogue
//   expert_swiglu        -- the same paired tile and SwiGLU, stored unquantized
//   expert_pair_partial  -- the paired tile's gate and up f32 partials per
//                           K-partition, into two outputs
//
// Work items are (expert, BM-row tile, BN-column block).  Each workgroup finds
// its (expert, tile) from a wave-level prefix over ceil(counts[e]/BM), the same
// enumeration the reference's tile map lists for that row tile
// (src/akas/ops/moe/kernel.py:79-118), so no host read of counts is needed and
// the launch stays graph-capturable.  The grid is the reference's capacity
// bound; surplus workgroups exit at once.
//
// Both kernels accumulate every (row, column) in one f32 register in ascending
// k-block order with acc = fma(P, as*ws, acc), so the fused gate/up values are
// bit-identical to two expert_partial calls and the fused codes to
// expert_partial x2 -> swiglu_experts -> quantize.
#include <algorithm>

#include "device_info.h"
#include "gemm_core.h"
#include "gemm_dma.h"
#include "moe_launch.h"
#include "quant_group.h"

namespace akas {

struct ExpertArgs {
  const uint8_t* x;    // activation codes: [r, k], [r*top, k] (routed) or packed rows
  const float* as;     // activation scales, same row indexing, k/128 per row
  const uint8_t* w;    // [E, N, K] codes (gate for the paired kernel)
  const void* ws;      // [E, NB, KB] block scales
  const uint8_t* w2;   // up codes (paired)
  const void* ws2;     // up block scales (paired)
  // An expert outside the bank: when xw is set, expert E-1 takes its codes
  // and scales from these ([N, K], [NB, KB]; xw2/xws2 the up half when
  // paired) and the bank holds experts 0 .. E-2.
  const uint8_t* xw;
  const void* xws;
  const uint8_t* xw2;
  const void* xws2;
  const int32_t* counts;
  const int32_t* routes;   // [E, r]
  const int32_t* offsets;  // expert_offsets (packed input/output)
  void* out;
  void* out2;          // up partials (expert_pair_partial)
  float* out_scales;
  // expert_combine: the routed_combine fold in the epilogue; the fused
  // route scan (SCAN kernels): the ids and active flags it scans
  const int32_t* ids;       // [r, top] expert ids (a rank is live when 0 <= id < E)
  const float* cweights;    // [r, top] combine weights
  const int32_t* active;    // [r] or null (every row active)
  int32_t* scan_counts;     // SCAN: counts [E] written for the later launches
  int32_t* scan_routes;     // SCAN: routes [E, r] written for the later launches
  // SCAN: columns of ids.  Below top, expert E-1 is the shared expert, routed
  // by every row at rank scan_cols, and ids name experts 0 .. E-2.
  int scan_cols;
  float* cout;              // [r, N] f32 combined rows
  int32_t* arrivals;        // [r, N / BN] per (row, column block) arrival counts
  int r, top, E, N, K;
  int x_rows;    // rows addressable in x / as (gathered rows are clamped to it)
  int out_rows;  // rows addressable in out (r*top, or packed rows)
  int routed, packed_in, packed_out;
  int parts, kb_per_part;
  int ws_dtype, prod_dtype, act_dtype;
  int max_tiles, tiles_n;
  int fair;  // progress-ordered wave priority in the k-loop (see expert_tiled_kernel)
};

// The work item of this workgroup: column block nb of row tile `tile` of
// expert `expert`, whose routed rows number `count` (counts[expert] capped at
// r).  Items are enumerated over the live row tiles only, column block
// fastest, before the XCD remap: the grid is sized for the most tiles the
// routes can produce, and a remap over the whole grid left the dead tail --
// up to a quarter of the grid -- on the last XCDs, idling them.
struct Item {
  int nb, expert, tile, count;
};

// Position of logical tile t among the row tiles n (one expert per lane) of
// experts e0 .. e0+63, whose tiles start at `base`: sets the item and
// returns true when t falls among them, else advances base.
AKAS_DEV bool tile_in_chunk(int n, int c, int e0, int t, int r, int lane, int& base, Item& it) {
  const int incl = wave_inclusive_scan(n, lane);
  const int excl = incl - n;
  const uint64_t hit = __ballot(t >= base + excl && t < base + incl);
  if (hit) {
    const int src = __builtin_ctzll(hit);
    it.expert = e0 + src;
    it.tile = t - base - __shfl(excl, src, 64);
    it.count = min(__shfl(c, src, 64), r);
    return true;
  }
  base += __shfl(incl, 63, 64);
  return false;
}

// Returns false for a workgroup past the live items (uniform).  Up to 64
// experts, counts is read once and the total and the search share those
// registers: one memory round trip, where separate passes and the count read
// again after them took three in series.  More experts read counts once per
// pass, 64 at a time.
// Up to 64 experts: c is lane e's count (0 past the experts).
AKAS_DEV bool find_item_64(int c, int r, int bm, int tiles_n, int lane, Item& it) {
  const int n = (c + bm - 1) / bm;
  const int items = wave_sum_i(n) * tiles_n;
  const int id = xcd_remap(blockIdx.x, items);
  if (id >= items) return false;
  it.nb = id % tiles_n;
  int base = 0;
  return tile_in_chunk(n, c, 0, id / tiles_n, r, lane, base, it);
}

AKAS_DEV bool find_item(const int32_t* counts, int experts, int r, int bm, int tiles_n, int lane,
                        Item& it) {
  if (experts <= 64)
    return find_item_64(lane < experts ? max(counts[lane], 0) : 0, r, bm, tiles_n, lane, it);
  int total = 0;
  for (int e0 = 0; e0 < experts; e0 += 64) {
    const int e = e0 + lane;
    const int c = e < experts ? max(counts[e], 0) : 0;
    total += wave_sum_i((c + bm - 1) / bm);
  }
  const int items = total * tiles_n;
  const int id = xcd_remap(blockIdx.x, items);
  if (id >= items) return false;
  it.nb = id % tiles_n;
  const int t = id / tiles_n;
  int base = 0;
  for (int e0 = 0; e0 < experts; e0 += 64) {
    const int e = e0 + lane;
    const int c = e < experts ? max(counts[e], 0) : 0;
    if (tile_in_chunk((c + bm - 1) / bm, c, e0, t, r, lane, base, it)) return true;
  }
  return false;  // not reached: t < total
}

// Codes and block scales of expert e: the bank's slice, or the expert kept
// outside the bank (its scale index then starts at expert 0).
struct ExpertSlice {
  const uint8_t* w;
  const uint8_t* w2;
  const void* ws;
  const void* ws2;
  int scale_expert;
};

AKAS_DEV ExpertSlice expert_slice(const ExpertArgs& p, int e) {
  ExpertSlice q;
  if (p.xw && e == p.E - 1) {
    q.w = p.xw; q.w2 = p.xw2; q.ws = p.xws; q.ws2 = p.xws2; q.scale_expert = 0;
  } else {
    const int64_t ebase = (int64_t)e * p.N * p.K;
    q.w = p.w + ebase; q.w2 = p.w2 ? p.w2 + ebase : nullptr; q.ws = p.ws; q.ws2 = p.ws2;
    q.scale_expert = e;
  }
  return q;
}

// Tile row `idx` of expert e (a position below its count): its source row
// in the activation buffer, clamped into the buffer (a corrupt route can
// only misroute, never fault), and, when `live`, its scatter destination
// (else -1).  The route is read once for both.
// tile_route issues the loads, tile_row_of uses them, so that loads issued
// in between stay in flight.
struct RowRoute {
  int route, off;
};

AKAS_DEV RowRoute tile_route(const ExpertArgs& p, int e, int idx) {
  RowRoute q{0, 0};
  if (!p.packed_in || !p.packed_out) q.route = p.routes[(int64_t)e * p.r + idx];
  if (p.packed_in || p.packed_out) q.off = p.offsets[e];
  return q;
}

AKAS_DEV void tile_row_of(const ExpertArgs& p, RowRoute q, int idx, bool live, int& src,
                          int& dst) {
  const int row = p.packed_in ? q.off + idx : (p.routed ? q.route : q.route / p.top);
  src = row < 0 ? 0 : (row >= p.x_rows ? p.x_rows - 1 : row);
  const int d = live ? (p.packed_out ? q.off + idx : q.route) : -1;
  dst = d < p.out_rows ? d : -1;
}

AKAS_DEV void tile_row(const ExpertArgs& p, int e, int idx, bool live, int& src, int& dst) {
  tile_row_of(p, tile_route(p, e, idx), idx, live, src, dst);
}

// ---------------------------------------------------------------------------
// The route scan fused into the decode gate/up launch (quantized_routes,
// src/akas/ops/moe/kernel.py:121-151, done by every workgroup for itself).
// Up to 512 experts and 4096 entries g = row * cols + rank of ids [r, cols]
// (cols = scan_cols): thread t of the 256 holds entries t + 256j, so each
// pass j reads 1 KB of ids in one coalesced load per wave (every workgroup of
// the launch reads the same lines; per-lane strided loads cost the launch
// 6 us).  An expert's route at position q is its q-th live entry in g order,
// and names the entry row * top + rank; counts[e] = min(entries, r), as the
// route tables hold at most r routes per expert.  With a shared expert
// (cols < top), expert E-1 routes every row at rank cols, in row order.
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanPasses = 16;
constexpr int kScanMaxEntries = kScanThreads * kScanPasses;
constexpr int kScanMaxExperts = 512;
constexpr int kScanMaxCols = 64;

// Row of entry g (g < 65536, cols <= 64): the high word of g * ceil(2^32/cols)
// equals g / cols over that whole range (checked exhaustively).
AKAS_DEV int scan_row(int g, uint32_t magic) {
  return magic ? (int)__umulhi((uint32_t)g, magic) : g;
}

// The route naming entry g: row * top + rank.
AKAS_DEV int scan_route(const ExpertArgs& p, int g, int row) {
  return g + row * (p.top - p.scan_cols);
}

// Entry t + 256j of this thread: its expert id, or -1 past the end, for an
// inactive row or an id outside the routed experts.  Every load is issued
// before the first is used.
AKAS_DEV void scan_entries(const ExpertArgs& p, int tid, uint32_t magic, int (&id)[kScanPasses]) {
  const int n = p.r * p.scan_cols;
  const unsigned routed = (unsigned)(p.scan_cols < p.top ? p.E - 1 : p.E);
  int raw[kScanPasses], act[kScanPasses];
#pragma unroll
  for (int j = 0; j < kScanPasses; ++j) {
    const int g = tid + kScanThreads * j;
    raw[j] = -1;
    act[j] = 1;
    if (g < n) {
      raw[j] = p.ids[g];
      if (p.active) act[j] = p.active[scan_row(g, magic)];
    }
  }
#pragma unroll
  for (int j = 0; j < kScanPasses; ++j)
    id[j] = ((act[j] != 0) & ((unsigned)raw[j] < routed)) ? raw[j] : -1;
}

// find_item over the counts in LDS (hist, capped at r).
AKAS_DEV bool find_item_hist(const int* hist, int experts, int r, int bm, int tiles_n, int lane,
                             Item& it) {
  if (experts <= 64)
    return find_item_64(lane < experts ? min(hist[lane], r) : 0, r, bm, tiles_n, lane, it);
  int total = 0;
  for (int e0 = 0; e0 < experts; e0 += 64) {
    const int e = e0 + lane;
    total += wave_sum_i(e < experts ? (min(hist[e], r) + bm - 1) / bm : 0);
  }
  const int items = total * tiles_n;
  const int id = xcd_remap(blockIdx.x, items);
  if (id >= items) return false;
  it.nb = id % tiles_n;
  const int t = id / tiles_n;
  int base = 0;
  for (int e0 = 0; e0 < experts; e0 += 64) {
    const int e = e0 + lane;
    const int c = e < experts ? min(hist[e], r) : 0;
    if (tile_in_chunk((c + bm - 1) / bm, c, e0, t, r, lane, base, it)) return true;
  }
  return false;  // not reached: t < total
}

// counts [E] (workgroup 0) and the -1 padding of routes [E, r] past each
// expert's count (expert e by workgroup e, e + grid, ...): the tables
// quantized_routes leaves, for the launches after this one.
AKAS_DEV void scan_tables(const ExpertArgs& p, const int* hist, int tid) {
  if (blockIdx.x == 0)
    for (int e = tid; e < p.E; e += kScanThreads) p.scan_counts[e] = min(hist[e], p.r);
  for (int e = blockIdx.x; e < p.E; e += gridDim.x) {
    int32_t* out = p.scan_routes + (int64_t)e * p.r;
    for (int i = min(hist[e], p.r) + tid; i < p.r; i += kScanThreads) out[i] = -1;
  }
}

// Rows row0 .. row0+BM-1 of expert e's routes (count of them live): source
// rows and scatter destinations into rows_src / rows_dst (rows past count
// repeat the first row's source and scatter nowhere), and, from column
// block 0's workgroup, the routes themselves into scan_routes.  A pass's
// matches are numbered by wave ballots and per-wave totals in LDS.
template <int BM>
AKAS_DEV void scan_tile_rows(const ExpertArgs& p, const int (&id)[kScanPasses], uint32_t magic,
                             int e, int row0, int count, bool write_routes, int tid,
                             int (*wave_count)[4], int* rows_src, int* rows_dst) {
  int32_t* routes = p.scan_routes + (int64_t)e * p.r;
  if (p.scan_cols < p.top && e == p.E - 1) {  // the shared expert (uniform)
    if (tid < BM) {
      const int pos = row0 + tid;
      const bool live = pos < count;
      const int route = pos * p.top + p.scan_cols;
      rows_src[tid] = live ? pos : row0;
      rows_dst[tid] = live ? route : -1;
      if (live && write_routes) routes[pos] = route;
    }
    return;
  }
  const int lane = tid & 63, wave = tid >> 6;
  const uint64_t below = (uint64_t{1} << lane) - 1;
  uint64_t hit[kScanPasses];
#pragma unroll
  for (int j = 0; j < kScanPasses; ++j) hit[j] = __ballot(id[j] == e);
  if (lane < kScanPasses) {
    uint64_t h = hit[0];
#pragma unroll
    for (int j = 1; j < kScanPasses; ++j) h = lane == j ? hit[j] : h;
    wave_count[lane][wave] = __builtin_popcountll(h);
  }
  __syncthreads();
  int done = 0;  // matches in the passes before j
#pragma unroll
  for (int j = 0; j < kScanPasses; ++j) {
    const int c0 = wave_count[j][0], c1 = wave_count[j][1], c2 = wave_count[j][2],
              c3 = wave_count[j][3];
    const int before = (wave > 0 ? c0 : 0) + (wave > 1 ? c1 : 0) + (wave > 2 ? c2 : 0);
    const int pos = done + before + __builtin_popcountll(hit[j] & below);
    if ((id[j] == e) & (pos >= row0) & (pos < row0 + BM) & (pos < count)) {
      const int g = tid + kScanThreads * j;
      const int src = scan_row(g, magic);
      const int f = scan_route(p, g, src);
      rows_src[pos - row0] = src;
      rows_dst[pos - row0] = f;
      if (write_routes) routes[pos] = f;
      if (pos == row0)
        for (int i = count - row0; i < BM; ++i) {
          rows_src[i] = src;
          rows_dst[i] = -1;
        }
    }
    done += c0 + c1 + c2 + c3;
  }
}

// Epilogue modes of the grouped kernels.  Modes 1-3 share the paired tile:
// B holds 16-row gate and up tiles interleaved, so each lane ends with the
// gate and the up value of the same (row, column).
enum ExpertMode {
  kPartial = 0,      // expert_partial: out[route][part][col] in OUT
  kSwigluFp8 = 1,    // fp8_expert_swiglu: SwiGLU, per-128 FP8 codes + scales
  kSwiglu = 2,       // expert_swiglu: SwiGLU stored in OUT
  kPairPartial = 3,  // expert_pair_partial: gate -> out, up -> out2, f32 per part
  kCombine = 4,      // expert_combine: kPartial's stores, then the rank-ordered fold
};

// Modes whose B tile holds gate and up rows.
constexpr bool paired_mode(int mode) { return mode == kSwigluFp8 || mode == kSwiglu || mode == kPairPartial; }

// Live ranks of row t: its ids inside [0, E) (the ranks quantized_routes
// routes when the row is active).
AKAS_DEV int live_ranks(const ExpertArgs& p, int t) {
  int n = 0;
  for (int k = 0; k < p.top; ++k) {
    const int e = p.ids[(int64_t)t * p.top + k];
    n += e >= 0 && e < p.E;
  }
  return n;
}

// expert_combine, rows no route reaches (inactive, or without a live rank):
// their combined row is zero.  Row t belongs to workgroup t % gridDim.x, so
// every workgroup of the grid, live or not, takes a share before its exit.
template <int THREADS>
AKAS_DEV void zero_unrouted_rows(const ExpertArgs& p) {
  for (int t = blockIdx.x; t < p.r; t += gridDim.x) {
    const bool routed = (!p.active || p.active[t] != 0) && live_ranks(p, t) > 0;  // uniform
    if (routed) continue;
    v4f* row = reinterpret_cast<v4f*>(p.cout + (int64_t)t * p.N);
    for (int c = threadIdx.x; c < p.N / 4; c += THREADS) row[c] = v4f{0.f, 0.f, 0.f, 0.f};
  }
}

// expert_combine tail, after the workgroup has stored its contributions
// (rows rows_dst[0..BM), columns n0 .. n0+BN) in CDT:
//   * release fence, then one arrival per live row on the counter of its
//     (token, column block); the arrival that completes the token's live
//     ranks (every other rank's workgroup has stored and fenced before its
//     own arrival) resets the counter to zero and takes the token;
//   * if the workgroup took any token: acquire fence, then the taken tokens'
//     combined columns: acc = 0, then acc = fma(contribution[token, rank],
//     weight[token, rank], acc) over the live ranks in rank order --
//     routed_combine's fold on the stored (rounded) contributions, so the
//     result is the same bit for bit.
// Exactly one arrival completes each counter, so no workgroup waits for
// another and the counters are left zero for the next call.  On gfx950 the
// device-scope release is an L2 write-back per workgroup (buffer_wbl2), the
// price of handing the contributions across XCDs inside one launch.
template <int BM, int BN, int THREADS, int CDT>
AKAS_DEV void combine_tail(const ExpertArgs& p, const int* rows_dst, int* taken, int* ntaken,
                           int nb, int n0) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if (threadIdx.x == 0) *ntaken = 0;
  __syncthreads();
  const int blocks = p.N / BN;
  for (int i = threadIdx.x; i < BM; i += THREADS) {
    const int dst = rows_dst[i];
    if (dst < 0) continue;
    const int t = dst / p.top;
    int32_t* counter = p.arrivals + (int64_t)t * blocks + nb;
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before + 1 == live_ranks(p, t)) {
      __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      taken[atomicAdd(ntaken, 1)] = t;  // LDS slot; the fold order is per token, not per slot
    }
  }
  __syncthreads();
  const int n = *ntaken;  // uniform
  if (n == 0) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  constexpr int G = BN / 4;  // four columns per thread
  for (int u = threadIdx.x; u < n * G; u += THREADS) {
    const int t = taken[u / G];
    const int col = n0 + 4 * (u % G);
    const int64_t row = (int64_t)t * p.top;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < p.top; ++k) {
      const int e = p.ids[row + k];
      if (e < 0 || e >= p.E) continue;
      const float w = p.cweights[row + k];
      const int64_t at = (row + k) * p.N + col;
      v4f v;
      if constexpr (CDT == AKAS_DTYPE_F32) {
        v = *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(p.out) + at);
      } else {
        const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.out) + at);
        if constexpr (CDT == AKAS_DTYPE_BF16) {
          v = v4f{bf16_bits_to_f32(h.x & 0xFFFFu), bf16_bits_to_f32(h.x >> 16),
                  bf16_bits_to_f32(h.y & 0xFFFFu), bf16_bits_to_f32(h.y >> 16)};
        } else {
          v = v4f{f16_bits_to_f32(h.x & 0xFFFFu), f16_bits_to_f32(h.x >> 16),
                  f16_bits_to_f32(h.y & 0xFFFFu), f16_bits_to_f32(h.y >> 16)};
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf(v[q], w, acc[q]);
    }
    *reinterpret_cast<v4f*>(p.cout + (int64_t)t * p.N + col) = acc;
  }
}

// Wave priority by the share of its k range a wave has done: 3 in the first
// quarter down to 0 in the last.  When all of a launch's workgroups are
// resident at once (one round, several per CU), the SIMDs otherwise favour
// the oldest workgroup's waves: of the three gate/up workgroups on a CU the
// first finished 20 us before the last (LFM2 decode layer, 768 workgroups),
// and the last ran its tail alone at a fraction of the CU's load rate.  A
// wave that lags keeps the higher priority until it has caught up to within
// a quarter (per-CU spread 20 -> 5 us, layer 134.0 -> 131.1 us).  With more
// workgroups than slots the oldest-first order is the better one: finished
// workgroups free their slots for the next ones.
AKAS_DEV void wave_priority_by_progress(int done, int total) {
  const int q = (done * 4) / total;  // wave-uniform
  if (q == 0)
    __builtin_amdgcn_s_setprio(3);
  else if (q == 1)
    __builtin_amdgcn_s_setprio(2);
  else if (q == 2)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

// STAGES: LDS stages (0: one for the 32-row expert partial, two otherwise).
// The one-stage paired 32-row tile keeps its registers within three waves per
// SIMD, so that three workgroups share a CU.
// SCAN: the workgroup scans ids itself (scan_entries) instead of reading the
// route tables, and writes them for the launches after it.
template <int BM, int BN, int WAVES_M, int WAVES_N, int MODE, int OUT, int SDT, int STAGES = 0,
          int SCAN = 0>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N)
__attribute__((amdgpu_waves_per_eu((STAGES == 1 && BM == 16 && paired_mode(MODE)) ? 4
                                   : (STAGES == 1 && BM == 32 && paired_mode(MODE)) ? 3 : 1)))
void expert_tiled_kernel(ExpertArgs p) {
  constexpr int THREADS = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int MT = WM / 16, NT = WN / 16;
  constexpr bool PAIRED = paired_mode(MODE);
  static_assert(!PAIRED || (BN == 256 && NT % 2 == 0), "paired tiles hold 128 gate + 128 up");
  static_assert(PAIRED || 128 % WN == 0, "a wave's columns must stay inside one scale block");
  using Plan = StagePlan<BM, BN, THREADS>;
  constexpr int STAGE = (BM + BN) * 128;
  // The 32-row expert partial (the decode down projection) keeps one LDS
  // stage, so that more workgroups share a CU: four instead of three with
  // 128 columns (20.9 KB; 38.6 -> 36.6 us at 64 experts x 1536 -> 2048), three
  // instead of two with 256 (36.9 KB; its registers then allow no more).  The
  // paired gate/up tile takes one stage (three workgroups per CU) only when
  // its launch asks for it (launch_paired).
  constexpr int NSTAGE = STAGES ? STAGES : ((!PAIRED && BM == 32) ? 1 : 2);
  __shared__ __attribute__((aligned(16))) uint8_t lds[NSTAGE * STAGE];
  __shared__ __attribute__((aligned(16))) float lds_as[NSTAGE][BM];
  __shared__ int rows_src[BM];
  __shared__ int rows_dst[BM];
  __shared__ float row_max[MODE == kSwigluFp8 ? WAVES_N : 1][MODE == kSwigluFp8 ? BM : 1];
  __shared__ int taken[MODE == kCombine ? BM : 1];
  __shared__ int ntaken;
  static_assert(!SCAN || THREADS == kScanThreads, "the route scan runs on 256 threads");
  __shared__ int scan_hist[SCAN ? kScanMaxExperts : 1];
  __shared__ int scan_wave[SCAN ? kScanPasses : 1][4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if constexpr (MODE == kCombine) zero_unrouted_rows<THREADS>(p);
  int sid[SCAN ? kScanPasses : 1];
  const uint32_t magic = p.scan_cols > 1 ? 0xFFFFFFFFu / (uint32_t)p.scan_cols + 1u : 0u;
  if constexpr (SCAN) {
    scan_entries(p, tid, magic, sid);
    for (int e = tid; e < p.E; e += THREADS) scan_hist[e] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kScanPasses; ++j)
      if (sid[j] >= 0) atomicAdd(&scan_hist[sid[j]], 1);
    if (p.scan_cols < p.top && tid == 0) scan_hist[p.E - 1] = p.r;  // the shared expert
    __syncthreads();
    scan_tables(p, scan_hist, tid);
  }
  // Live items first, then the XCD remap (as in the prefill kernel): the
  // workgroups of the capacity-sized grid that find no tile come last and
  // exit, so the live ones spread evenly over the CUs.  Column block fastest:
  // neighbouring workgroups read one expert's consecutive weight rows and
  // share its activation rows (LFM2 decode layer 145.5 -> 142.6 us, Qwen3.5
  // block 190.5 -> 183.2 us against tiles fastest over the whole grid).
  Item item;
  if constexpr (SCAN) {
    if (!find_item_hist(scan_hist, p.E, p.r, BM, p.tiles_n, lane, item)) return;  // uniform
  } else if (!find_item(p.counts, p.E, p.r, BM, p.tiles_n, lane, item)) {
    return;  // uniform
  }
  const int nb = item.nb, e = item.expert, tile = item.tile, count = item.count;
  const int row0 = tile * BM;
  if (row0 >= count) return;  // only reachable with counts[e] > r
  const int n0 = nb * (PAIRED ? BN / 2 : BN);
  const int part = blockIdx.y;
  const int KB = p.K / kBlock, NB = (p.N + kBlock - 1) / kBlock;
  const int kb0 = part * p.kb_per_part, kb1 = kb0 + p.kb_per_part;

  const ExpertSlice xs = expert_slice(p, e);

  Plan plan;
  u32x4 ra[Plan::CA], rb[Plan::CB];
  const int prow = tid >> 3, pch = tid & 7;
  {
    const int row = prow, ch = pch;
    if constexpr (PAIRED) {
      // B row rho: 16-row tile j = rho/16 is gate (even j) or up (odd j)
      // column n0 + (rho/32)*16 + rho%16; the parity is fixed per thread.
      const bool up = (row >> 4) & 1;
      plan.b_base = up ? xs.w2 : xs.w;
      plan.b_off = (uint32_t)(n0 + (row >> 5) * 16 + (row & 15)) * (uint32_t)p.K + ch * 16;
      plan.b_step = (uint32_t)(Plan::RSTEP / 2) * (uint32_t)p.K;
    } else {
      plan.b_base = xs.w;
      plan.b_off = (uint32_t)(n0 + row) * (uint32_t)p.K + ch * 16;
      plan.b_step = (uint32_t)Plan::RSTEP * (uint32_t)p.K;
    }
    plan.dst0 = lds_off(row, ch);
  }
  // Gathered source rows and scatter destinations of this tile.  The first
  // weight k-block is requested before they are known: after the route
  // loads, or before the route scan's barriers, which then run under it.
  if constexpr (SCAN) {
    plan.fetch_b(kb0, rb);
    scan_tile_rows<BM>(p, sid, magic, e, row0, count, nb == 0, tid, scan_wave, rows_src,
                       rows_dst);
  } else {
    static_assert(BM <= THREADS, "one tile row per thread");
    const int idx = row0 + tid;
    const bool live = idx < count;
    RowRoute q{0, 0};
    if (tid < BM) q = tile_route(p, e, live ? idx : row0);
    plan.fetch_b(kb0, rb);
    if (tid < BM) tile_row_of(p, q, live ? idx : row0, live, rows_src[tid], rows_dst[tid]);
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < Plan::CA; ++i)
    plan.a_off[i] = (uint32_t)rows_src[min(prow + i * Plan::RSTEP, BM - 1)] * (uint32_t)p.K + pch * 16;
  plan.a_live = prow < BM;
  plan.a_base = p.x;
  const float* as_row = p.as + (int64_t)rows_src[tid < BM ? tid : 0] * KB;

  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int a_row0 = wm * WM, b_row0 = wn * WN;
  // Scale block of this wave's columns (gate and up share it when paired).
  const int wcol = PAIRED ? n0 + b_row0 / 2 : n0 + b_row0;
  const int64_t ws_base = ((int64_t)xs.scale_expert * NB + wcol / kBlock) * KB;

  Acc<MT, NT> acc;
  acc.clear();
  // Every global load (data and both scales) is issued one k-block before its
  // use: loads complete in issue order, so a scale fetched after the
  // prefetch would make the current multiply wait for that prefetch.
  float ras, rws0, rws1 = 0.f;
  if constexpr (NSTAGE == 1) {
    // one stage: stash, prefetch the next k-block, barrier, multiply, barrier
    plan.fetch_a(kb0, ra);
    ras = as_row[kb0];
    rws0 = load_scale_t<SDT>(xs.ws, ws_base + kb0);
    if constexpr (PAIRED) rws1 = load_scale_t<SDT>(xs.ws2, ws_base + kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
      if constexpr (STAGES == 1)
        if (p.fair) wave_priority_by_progress(kb - kb0, kb1 - kb0);
      if (kb > kb0) __syncthreads();  // the previous multiply is done with the stage
      plan.stash(lds, ra, rb);
      if (tid < BM) lds_as[0][tid] = ras;
      const float ws0 = rws0, ws1 = rws1;
      const int nxt = min(kb + 1, kb1 - 1);
      plan.fetch(nxt, ra, rb);
      ras = as_row[nxt];
      rws0 = load_scale_t<SDT>(xs.ws, ws_base + nxt);
      if constexpr (PAIRED) rws1 = load_scale_t<SDT>(xs.ws2, ws_base + nxt);
      __syncthreads();
      mma_stage<MT, NT, PAIRED>(acc, lds, lds + BM * 128, lds_as[0], a_row0, b_row0, ws0, lane, ws1);
    }
    __syncthreads();
  } else {
    plan.fetch_a(kb0, ra);
    ras = as_row[kb0];
    float ws0 = load_scale_t<SDT>(xs.ws, ws_base + kb0);
    float ws1 = PAIRED ? load_scale_t<SDT>(xs.ws2, ws_base + kb0) : 0.f;
    plan.stash(lds, ra, rb);
    if (tid < BM) lds_as[0][tid] = ras;
    {
      const int nxt = min(kb0 + 1, kb1 - 1);
      plan.fetch(nxt, ra, rb);
      ras = as_row[nxt];
      rws0 = load_scale_t<SDT>(xs.ws, ws_base + nxt);
      if constexpr (PAIRED) rws1 = load_scale_t<SDT>(xs.ws2, ws_base + nxt);
    }
    __syncthreads();

    for (int kb = kb0; kb < kb1; ++kb) {
      const int cur = (kb - kb0) & 1;
      mma_stage<MT, NT, PAIRED>(acc, lds + cur * STAGE, lds + cur * STAGE + BM * 128, lds_as[cur],
                                a_row0, b_row0, ws0, lane, ws1);
      plan.stash(lds + (cur ^ 1) * STAGE, ra, rb);
      if (tid < BM) lds_as[cur ^ 1][tid] = ras;
      ws0 = rws0;
      ws1 = rws1;
      const int nxt = min(kb + 2, kb1 - 1);
      plan.fetch(nxt, ra, rb);
      ras = as_row[nxt];
      rws0 = load_scale_t<SDT>(xs.ws, ws_base + nxt);
      if constexpr (PAIRED) rws1 = load_scale_t<SDT>(xs.ws2, ws_base + nxt);
      __syncthreads();
    }
  }

  if constexpr (!PAIRED) {
    const int64_t rstride = (int64_t)p.parts * p.N;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int lr = a_row0 + 16 * i + 4 * (lane >> 4) + e4;
        const int dst = rows_dst[lr];
        if (dst < 0) continue;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int col = wcol + 16 * j + (lane & 15);
          store_out<OUT>(p.out, (int64_t)dst * rstride + (int64_t)part * p.N + col,
                         acc.t[i][j][e4]);
        }
      }
    if constexpr (MODE == kCombine) combine_tail<BM, BN, THREADS, OUT>(p, rows_dst, taken, &ntaken, nb, n0);
  } else if constexpr (MODE == kPairPartial) {
    const int64_t rstride = (int64_t)p.parts * p.N;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int dst = rows_dst[a_row0 + 16 * i + 4 * (lane >> 4) + e4];
        if (dst < 0) continue;
#pragma unroll
        for (int j = 0; j < NT / 2; ++j) {
          const int64_t at = (int64_t)dst * rstride + (int64_t)part * p.N + wcol + 16 * j + (lane & 15);
          reinterpret_cast<float*>(p.out)[at] = acc.t[i][2 * j][e4];
          reinterpret_cast<float*>(p.out2)[at] = acc.t[i][2 * j + 1][e4];
        }
      }
  } else if constexpr (MODE == kSwiglu) {
    with_dtype(p.prod_dtype, [&](auto PD) __attribute__((always_inline)) {
      with_dtype(p.act_dtype, [&](auto AD) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const int dst = rows_dst[a_row0 + 16 * i + 4 * (lane >> 4) + e4];
            if (dst < 0) continue;
#pragma unroll
            for (int j = 0; j < NT / 2; ++j) {
              const float g = round_t<decltype(PD)::value>(acc.t[i][2 * j][e4]);
              const float u = round_t<decltype(PD)::value>(acc.t[i][2 * j + 1][e4]);
              const float a = round_t<decltype(AD)::value>(swiglu_elem(g, u));
              store_out<OUT>(p.out, (int64_t)dst * p.N + wcol + 16 * j + (lane & 15), a);
            }
          }
      });
    });
  } else {
    // SwiGLU on (gate, up) pairs held by the same lane, then row max over the
    // 128 activation columns of the tile (16 lanes x NT/2 tiles x WAVES_N).
    float act[MT][NT / 2][4];
    float rmax[MT][4];
    with_dtype(p.prod_dtype, [&](auto PD) __attribute__((always_inline)) {
      with_dtype(p.act_dtype, [&](auto AD) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            float m = 0.f;
#pragma unroll
            for (int j = 0; j < NT / 2; ++j) {
              const float g = round_t<decltype(PD)::value>(acc.t[i][2 * j][e4]);
              const float u = round_t<decltype(PD)::value>(acc.t[i][2 * j + 1][e4]);
              const float a = round_t<decltype(AD)::value>(swiglu_elem(g, u));
              act[i][j][e4] = a;
              m = __builtin_fmaxf(m, __builtin_fabsf(a));
            }
            rmax[i][e4] = m;
          }
      });
    });
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        rmax[i][e4] = row16_max(rmax[i][e4]);
      }
    if ((lane & 15) == 0) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) row_max[wn][a_row0 + 16 * i + 4 * (lane >> 4) + e4] = rmax[i][e4];
    }
    __syncthreads();
    uint8_t* codes = reinterpret_cast<uint8_t*>(p.out);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int lr = a_row0 + 16 * i + 4 * (lane >> 4) + e4;
        float m = row_max[0][lr];
#pragma unroll
        for (int w = 1; w < WAVES_N; ++w) m = __builtin_fmaxf(m, row_max[w][lr]);
        const GroupScale gs = make_group_scale(m);
        const int dst = rows_dst[lr];
        if (dst < 0) continue;
#pragma unroll
        for (int j = 0; j < NT / 2; ++j) {
          const int col = wcol + 16 * j + (lane & 15);
          codes[(int64_t)dst * p.N + col] = (uint8_t)e4m3_encode_scaled(act[i][j][e4], gs);
        }
        if (wn == 0 && (lane & 15) == 0) p.out_scales[(int64_t)dst * (p.N / kBlock) + n0 / kBlock] = gs.s;
      }
  }
}

// ---------------------------------------------------------------------------
// Prefill-sized experts: 256-row tiles on the DMA-fed 256x256 tile engine
// (gemm_dma.h).  Waves 0-3 gather their A rows through the tile's route
// table; waves 4-7 copy weight rows (MODE 1: gate rows for pieces 0,1,4,5
// and up rows for pieces 2,3,6,7, i.e. 16-row gate/up tiles interleaved).
// Work items are walked column block fastest, so a row tile's activations
// stay in L2 across its column blocks and neighbouring row tiles of one
// expert share its weights.
// ---------------------------------------------------------------------------
template <int MODE, int OUT>
__global__ __launch_bounds__(dma::THREADS) void expert_dma_kernel(ExpertArgs p) {
  constexpr bool PAIRED = paired_mode(MODE);
  constexpr int BM = dma::BM;
  __shared__ int rows_src[BM];
  __shared__ int rows_dst[BM];
  __shared__ float row_max[MODE == kSwigluFp8 ? 2 : 1][MODE == kSwigluFp8 ? BM : 1];
  __shared__ int taken[MODE == kCombine ? BM : 1];
  __shared__ int ntaken;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if constexpr (MODE == kCombine) zero_unrouted_rows<dma::THREADS>(p);
  Item item;
  if (!find_item(p.counts, p.E, p.r, BM, p.tiles_n, lane, item)) return;  // uniform
  const int nb = item.nb, e = item.expert, tile = item.tile, count = item.count;
  const int row0 = tile * BM;
  if (row0 >= count) return;  // only reachable with counts[e] > r
  const int n0 = nb * (PAIRED ? dma::BN / 2 : dma::BN);
  const int part = blockIdx.y;
  const int KB = p.K / kBlock, NB = (p.N + kBlock - 1) / kBlock;
  const int kb0 = part * p.kb_per_part, kb1 = kb0 + p.kb_per_part;

  const ExpertSlice xs = expert_slice(p, e);
  // Weight scales over the k range as float32 (either scale dtype gives the
  // same main loop): PAIRED, gate (h = 0) and up (h = 1) of the tile's one
  // 128-column block; else the tile's two column blocks.  One scale and one
  // tile row per thread; every load is issued before the first LDS store,
  // so the scales and the routes take one memory round trip together.
  static_assert(BM <= dma::THREADS && 2 * dma::MAX_KB <= dma::THREADS, "one entry per thread");
  // (The scale's raw bits are widened only after the route loads are out.)
  const int nkb = kb1 - kb0;
  uint32_t wraw = 0;
  if (tid < 2 * nkb) {
    const int h = tid / nkb, k = kb0 + tid % nkb;
    const void* src = (PAIRED && h) ? xs.ws2 : xs.ws;
    const int cb = PAIRED ? n0 / kBlock : min((n0 + 128 * h) / kBlock, NB - 1);
    const int64_t at = ((int64_t)xs.scale_expert * NB + cb) * KB + k;
    wraw = p.ws_dtype == AKAS_DTYPE_F32 ? reinterpret_cast<const uint32_t*>(src)[at]
                                        : reinterpret_cast<const uint16_t*>(src)[at];
  }
  int src_row = 0, dst_row = -1;
  if (tid < BM) {
    const int idx = row0 + tid;
    const bool live = idx < count;
    tile_row(p, e, live ? idx : row0, live, src_row, dst_row);
  }
  if (tid < BM) {
    rows_src[tid] = src_row;
    rows_dst[tid] = dst_row;
  }
  if (tid < 2 * nkb)
    dma::wtab[tid / nkb][tid % nkb] = __uint_as_float(p.ws_dtype == AKAS_DTYPE_F32 ? wraw : wraw << 16);
  __syncthreads();

  dma::GatherPlan plan;
  plan.blk0 = wave * 8;
  plan.as = p.as;
  if (wave < 4) {
    plan.src = p.x;
    plan.alt_delta = 0;
    plan.alt_mask = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = dma::piece_row(wave, i, lane);
      plan.off[i] = (uint32_t)rows_src[row] * (uint32_t)p.K + dma::piece_chunk(row, lane);
    }
    plan.soff = (uint32_t)rows_src[(wave & 3) * 64 + lane] * (uint32_t)KB;
    plan.scales = true;
    plan.skip = row0 + (wave & 3) * 64 >= count;  // a quarter of padding rows only
  } else {
    plan.src = xs.w;
    plan.alt_delta = PAIRED ? (int64_t)(xs.w2 - xs.w) : 0;
    plan.alt_mask = PAIRED ? 0xCCu : 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rho = dma::piece_row(wave, i, lane);
      const int col = PAIRED ? n0 + (rho >> 5) * 16 + (rho & 15) : n0 + rho;
      plan.off[i] = (uint32_t)col * (uint32_t)p.K + dma::piece_chunk(rho, lane);
    }
    plan.soff = 0;
    plan.scales = false;
    plan.skip = false;
  }

  const int wm = wave & 3, wn = wave >> 2;
  const int a_row0 = wm * 64, b_row0 = wn * 128;
  // First output column of this wave; gate and up share its scale block.
  const int wcol = PAIRED ? n0 + b_row0 / 2 : n0 + b_row0;
  const float* w0 = dma::wtab[PAIRED ? 0 : wn];
  const float* w1 = dma::wtab[1];
  dma::Acc acc;
  acc.clear();
  dma::run<PAIRED>(plan, acc, a_row0, b_row0, kb0, kb1, lane, [&](int kb) {
    return float2{w0[kb - kb0], PAIRED ? w1[kb - kb0] : 0.f};
  }, row0 + a_row0 < count);  // a wave whose 64 rows are all padding only copies

  if constexpr (!PAIRED) {
    const int64_t rstride = (int64_t)p.parts * p.N;
    dma::store_tile<OUT>(
        acc, p.out, wave, lane, [&](int r) { return rows_dst[a_row0 + r] >= 0; },
        [&](int r) { return (int64_t)rows_dst[a_row0 + r] * rstride + (int64_t)part * p.N + wcol; });
    if constexpr (MODE == kCombine) combine_tail<BM, dma::BN, dma::THREADS, OUT>(p, rows_dst, taken, &ntaken, nb, n0);
  } else if constexpr (MODE == kPairPartial) {
    // Lane l holds, for m-tile i and column group c (0..3), gate in n-tile
    // 2c and up in n-tile 2c+1 of row a_row0 + 16i + l%16 at output columns
    // wcol + 16c + 4*(l/16) + 0..3: one 16-byte store into each output.
    const int64_t rstride = (int64_t)p.parts * p.N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int dst = rows_dst[a_row0 + 16 * i + (lane & 15)];
      if (dst < 0) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t at = (int64_t)dst * rstride + (int64_t)part * p.N + wcol + 16 * c + 4 * (lane >> 4);
        *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + at) = acc.t[i][2 * c];
        *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out2) + at) = acc.t[i][2 * c + 1];
      }
    }
  } else if constexpr (MODE == kSwiglu) {
    // Lane layout as above; SwiGLU of each (gate, up) pair, four adjacent
    // output columns per store.
    with_dtype(p.prod_dtype, [&](auto PD) __attribute__((always_inline)) {
      with_dtype(p.act_dtype, [&](auto AD) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dst = rows_dst[a_row0 + 16 * i + (lane & 15)];
          if (dst < 0) continue;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v4f a;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float g = round_t<decltype(PD)::value>(acc.t[i][2 * c][q]);
              const float u = round_t<decltype(PD)::value>(acc.t[i][2 * c + 1][q]);
              a[q] = round_t<decltype(AD)::value>(swiglu_elem(g, u));
            }
            store_out4<OUT>(p.out, (int64_t)dst * p.N + wcol + 16 * c + 4 * (lane >> 4), a);
          }
        }
      });
    });
  } else {
    // Lane l holds, for m-tile i and column group c (0..3), gate in n-tile
    // 2c and up in n-tile 2c+1 of row a_row0 + 16i + l%16 at output columns
    // wcol + 16c + 4*(l/16) + 0..3.  SwiGLU in place of the gate values, then
    // the row maximum over the tile's 128 output columns: 16 per lane group,
    // 4 lane groups (xor 16, 32), 2 waves (LDS).
    float rmax[4];
    with_dtype(p.prod_dtype, [&](auto PD) __attribute__((always_inline)) {
      with_dtype(p.act_dtype, [&](auto AD) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float m = 0.f;
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float g = round_t<decltype(PD)::value>(acc.t[i][2 * c][q]);
              const float u = round_t<decltype(PD)::value>(acc.t[i][2 * c + 1][q]);
              const float a = round_t<decltype(AD)::value>(swiglu_elem(g, u));
              acc.t[i][2 * c][q] = a;
              m = __builtin_fmaxf(m, __builtin_fabsf(a));
            }
          rmax[i] = m;
        }
      });
    });
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float m = __builtin_fmaxf(rmax[i], __shfl_xor(rmax[i], 16, 64));
      m = __builtin_fmaxf(m, __shfl_xor(m, 32, 64));
      if (lane < 16) row_max[wn][a_row0 + 16 * i + lane] = m;
    }
    __syncthreads();
    uint8_t* codes = reinterpret_cast<uint8_t*>(p.out);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = a_row0 + 16 * i + (lane & 15);
      const GroupScale gs = make_group_scale(__builtin_fmaxf(row_max[0][r], row_max[1][r]));
      const int dst = rows_dst[r];
      if (dst < 0) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const v4f& a = acc.t[i][2 * c];
        *reinterpret_cast<uint32_t*>(codes + (int64_t)dst * p.N + wcol + 16 * c + 4 * (lane >> 4)) =
            e4m3_encode4_scaled(a[0], a[1], a[2], a[3], gs);
      }
      if (wn == 0 && lane < 16) p.out_scales[(int64_t)dst * (p.N / kBlock) + n0 / kBlock] = gs.s;
    }
  }
}

// ---------------------------------------------------------------------------
// fp8_experts' group tables (moe_groups: experts [r*top], routes [r*top, r]
// holding a rank or -1) -> the grouped kernels' per-expert counts and routes
// (row*top + rank, in row order).  One workgroup per expert finds the group
// that owns it (each expert has at most one) and compacts that group's route
// row by an ordered block scan; an expert no group owns gets count 0.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void groups_to_routes_kernel(const int32_t* __restrict__ group_experts,
                                                               const int32_t* __restrict__ group_routes,
                                                               int32_t* __restrict__ counts,
                                                               int32_t* __restrict__ routes,
                                                               int64_t rows, int top) {
  __shared__ int owner;
  __shared__ int wave_tot[4];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) owner = 0x7FFFFFFF;
  __syncthreads();
  const int64_t groups = rows * top;
  for (int64_t g = tid; g < groups; g += 256)
    if (group_experts[g] == e) atomicMin(&owner, (int)g);
  __syncthreads();
  const int g = owner;  // uniform
  int32_t* out = routes + (int64_t)e * rows;
  int64_t base = 0;
  if (g != 0x7FFFFFFF) {
    const int32_t* row = group_routes + (int64_t)g * rows;
    for (int64_t b0 = 0; b0 < rows; b0 += 256) {
      const int64_t b = b0 + tid;
      const int rank = b < rows ? row[b] : -1;
      const int live = rank >= 0 && rank < top;
      const int incl = wave_inclusive_scan(live, lane);
      if (lane == 63) wave_tot[wave] = incl;
      __syncthreads();
      int before = 0, total = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        before += w < wave ? wave_tot[w] : 0;
        total += wave_tot[w];
      }
      if (live) out[base + before + incl - 1] = (int32_t)(b * top + rank);
      base += total;
      __syncthreads();
    }
  }
  if (tid == 0) counts[e] = (int32_t)base;
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------

int64_t capacity_tiles(int64_t r, int64_t top, int64_t experts, int64_t bm) {
  const int64_t routes = r * top;
  const int64_t b = (routes + bm - 1) / bm + experts - 1;
  return routes < b ? routes : b;
}

template <int BM, int BN, int WMW, int WNW, int MODE, int OUT, int STAGES = 0, int SCAN = 0>
static void launch_expert(ExpertArgs a, hipStream_t s) {
  a.max_tiles = (int)capacity_tiles(a.r, a.top, a.E, BM);
  a.tiles_n = paired_mode(MODE) ? a.N / (BN / 2) : a.N / BN;
  dim3 grid((unsigned)(a.max_tiles * a.tiles_n), (unsigned)a.parts);
  if (a.ws_dtype == AKAS_DTYPE_F32)
    expert_tiled_kernel<BM, BN, WMW, WNW, MODE, OUT, AKAS_DTYPE_F32, STAGES, SCAN>
        <<<grid, 64 * WMW * WNW, 0, s>>>(a);
  else
    expert_tiled_kernel<BM, BN, WMW, WNW, MODE, OUT, AKAS_DTYPE_BF16, STAGES, SCAN>
        <<<grid, 64 * WMW * WNW, 0, s>>>(a);
}

template <int MODE, int OUT>
static void launch_expert_dma(ExpertArgs a, hipStream_t s) {
  a.max_tiles = (int)capacity_tiles(a.r, a.top, a.E, dma::BM);
  a.tiles_n = paired_mode(MODE) ? a.N / (dma::BN / 2) : a.N / dma::BN;
  dim3 grid((unsigned)(a.max_tiles * a.tiles_n), (unsigned)a.parts);
  expert_dma_kernel<MODE, OUT><<<grid, dma::THREADS, 0, s>>>(a);
}

// Experts holding hundreds of rows on average (prefill batches) take the
// DMA-fed 256-row tiles; its 16-byte stores need a 16-byte aligned output.
static bool expert_dma_fits(const ExpertArgs& a, int64_t mean, int64_t n_mult) {
  return mean >= 128 && a.N % n_mult == 0 && a.kb_per_part <= dma::MAX_KB &&
         reinterpret_cast<uintptr_t>(a.out) % 16 == 0;
}

// Row tile by the mean rows per expert: 32-row tiles for decode-like batches,
// 128-row tiles in between, DMA-fed 256-row tiles for prefill batches.
template <int OUT, int MODE = kPartial>
static void launch_partial(const ExpertArgs& a, hipStream_t s) {
  const int64_t mean = (int64_t)a.r * a.top / a.E;
  // 256-column tiles where N allows: half the workgroups of 128-column ones,
  // each streaming twice the weights (LFM2 decode layer 146.0 -> 145.0 us,
  // the Qwen3.5 block 191.9 -> 189.2 us; 512 columns was slower).
  if (mean <= 48 && a.N % 256 == 0)
    launch_expert<32, 256, 1, 4, MODE, OUT>(a, s);
  else if (mean <= 48)
    launch_expert<32, 128, 1, 4, MODE, OUT>(a, s);
  else if (expert_dma_fits(a, mean, dma::BN))
    launch_expert_dma<MODE, OUT>(a, s);
  else
    launch_expert<128, 128, 2, 2, MODE, OUT>(a, s);
}

// The paired kernels (modes 1-3), row tile by the mean rows per expert as
// for expert_partial.  SCAN (the fused route scan) only where scan_fits
// holds, which keeps it to the tiled kernels below 49 mean rows.
template <int MODE, int OUT, int SCAN = 0>
static void launch_paired(const ExpertArgs& a, hipStream_t s) {
  const int64_t mean = (int64_t)a.r * a.top / a.E;
  const bool aligned = MODE != kPairPartial || reinterpret_cast<uintptr_t>(a.out2) % 16 == 0;
  // Decode batches: about one 32-row tile per active expert, at most
  // min(E, r*top) of them per column block.  When all of those workgroups fit
  // on the GPU at three per CU, the one-stage tile that allows three runs them
  // in a single round (LFM2 decode layer, 768 workgroups on 256 CUs: 142.9 ->
  // 135.5 us); when they do not, the two-stage tile's faster workgroups win
  // (Qwen3.5 block, about 900 workgroups: 184.0 against 191.4 us one-stage).
  const int64_t decode_tiles = std::min<int64_t>(a.E, (int64_t)a.r * a.top) * (a.N / 128) * a.parts;
  if (mean <= 8 && decode_tiles <= 4 * (int64_t)device_cus() + device_cus() / 4) {
    // a few rows per expert: 16-row tiles, four workgroups per CU
    ExpertArgs b = a;
    b.fair = decode_tiles >= 2 * (int64_t)device_cus();
    launch_expert<16, 256, 1, 4, MODE, OUT, 1, SCAN>(b, s);
  } else if (mean <= 48 && decode_tiles <= 3 * (int64_t)device_cus()) {
    // one round: progress-ordered priority once workgroups share CUs
    ExpertArgs b = a;
    b.fair = decode_tiles >= 2 * (int64_t)device_cus();
    launch_expert<32, 256, 1, 4, MODE, OUT, 1, SCAN>(b, s);
  } else if (mean <= 48) {
    launch_expert<32, 256, 1, 4, MODE, OUT, 0, SCAN>(a, s);
  } else if constexpr (!SCAN) {
    if (aligned && expert_dma_fits(a, mean, dma::BN / 2))
      launch_expert_dma<MODE, OUT>(a, s);
    else
      launch_expert<128, 256, 2, 4, MODE, OUT>(a, s);
  }
}

static void launch_swiglu(const ExpertArgs& a, hipStream_t s) {
  launch_paired<kSwigluFp8, AKAS_DTYPE_F32>(a, s);
}

// Shapes the fused route scan covers: a decode batch's routes (at least one
// row, up to 4096 entries of ids [r, cols], cols <= 64, at most 48 routes per
// expert on average over the launch's top ranks) over up to 512 experts.
static bool scan_fits(int64_t r, int cols, int top, int experts) {
  const int64_t n = r * cols;
  return r >= 1 && cols <= kScanMaxCols && experts <= kScanMaxExperts &&
         n <= kScanMaxEntries && r * top / experts <= 48;
}

static inline bool float_dtype(int d) {
  return d == AKAS_DTYPE_F32 || d == AKAS_DTYPE_F16 || d == AKAS_DTYPE_BF16;
}
static inline bool scale_dtype_ok(int d) { return d == AKAS_DTYPE_F32 || d == AKAS_DTYPE_BF16; }
static inline bool valid_block(int m) {
  return m == 4 || m == 8 || m == 16 || m == 32 || m == 64 || m == 128;
}

static int check_common(int64_t r, int top, int experts, int64_t o, int64_t k, int max_block_m,
                        int packed, int64_t x_rows) {
  if (r < 0 || top < 1 || experts < 1 || experts > 1024 || o <= 0 || k <= 0 || o % kBlock ||
      k % kBlock || !valid_block(max_block_m))
    return AKAS_ERR_GEOMETRY;
  if (r * top > 0x7FFFFFFF || o > 0x7FFFFFFF || k > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  if ((uint64_t)x_rows * (uint64_t)k >= (1ull << 32)) return AKAS_ERR_GEOMETRY;
  if ((uint64_t)o * (uint64_t)k >= (1ull << 32)) return AKAS_ERR_GEOMETRY;
  (void)packed;
  return AKAS_OK;
}

}  // namespace akas

using namespace akas;

extern "C" int akas_expert_partial(const uint8_t* x, const float* activation_scales,
                                   const uint8_t* w, const void* w_scales, int scale_dtype,
                                   const int32_t* counts, const int32_t* routes,
                                   const int32_t* tile_experts, const int32_t* tile_offsets,
                                   const int32_t* expert_offsets, void* out, int out_dtype,
                                   int64_t r, int top, int experts, int64_t o, int64_t k,
                                   int routed_input, int partitions, int max_block_m,
                                   int packed_input, void* stream) {
  (void)tile_experts;
  (void)tile_offsets;
  const int64_t x_rows = packed_input ? capacity_tiles(r, top, experts, max_block_m) * max_block_m
                                      : (routed_input ? r * top : r);
  int st = check_common(r, top, experts, o, k, max_block_m, packed_input, x_rows);
  if (st != AKAS_OK) return st;
  if (partitions < 1 || (k / kBlock) % partitions) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(out_dtype) || !scale_dtype_ok(scale_dtype)) return AKAS_ERR_DTYPE;
  if (partitions > 1 && out_dtype != AKAS_DTYPE_F32) return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !activation_scales || !w || !w_scales || !counts || !routes || !out)
    return AKAS_ERR_NULL;
  if (packed_input && !expert_offsets) return AKAS_ERR_NULL;
  ExpertArgs a{};
  a.x = x; a.as = activation_scales; a.w = w; a.ws = w_scales;
  a.counts = counts; a.routes = routes; a.offsets = expert_offsets; a.out = out;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.routed = routed_input; a.packed_in = packed_input; a.packed_out = 0;
  a.x_rows = (int)x_rows; a.out_rows = (int)(r * top);
  a.parts = partitions; a.kb_per_part = (int)(k / kBlock / partitions);
  a.ws_dtype = scale_dtype;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case AKAS_DTYPE_F32: launch_partial<AKAS_DTYPE_F32>(a, s); break;
    case AKAS_DTYPE_BF16: launch_partial<AKAS_DTYPE_BF16>(a, s); break;
    default: launch_partial<AKAS_DTYPE_F16>(a, s);
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_expert_combine(const uint8_t* x, const float* activation_scales,
                                   const uint8_t* w, const void* w_scales, int scale_dtype,
                                   const int32_t* counts, const int32_t* routes,
                                   const int32_t* expert_offsets, const int32_t* ids,
                                   const float* weights, const int32_t* active,
                                   void* contributions, int contribution_dtype, float* out,
                                   int32_t* arrivals, int64_t r, int top, int experts, int64_t o,
                                   int64_t k, int routed_input, int max_block_m, int packed_input,
                                   void* stream) {
  const int64_t x_rows = packed_input ? capacity_tiles(r, top, experts, max_block_m) * max_block_m
                                      : (routed_input ? r * top : r);
  int st = check_common(r, top, experts, o, k, max_block_m, packed_input, x_rows);
  if (st != AKAS_OK) return st;
  if (!float_dtype(contribution_dtype) || !scale_dtype_ok(scale_dtype)) return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !activation_scales || !w || !w_scales || !counts || !routes || !ids || !weights ||
      !contributions || !out || !arrivals)
    return AKAS_ERR_NULL;
  if (packed_input && !expert_offsets) return AKAS_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(contributions) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return AKAS_ERR_GEOMETRY;
  ExpertArgs a{};
  a.x = x; a.as = activation_scales; a.w = w; a.ws = w_scales;
  a.counts = counts; a.routes = routes; a.offsets = expert_offsets; a.out = contributions;
  a.ids = ids; a.cweights = weights; a.active = active; a.cout = out; a.arrivals = arrivals;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.routed = routed_input; a.packed_in = packed_input; a.packed_out = 0;
  a.x_rows = (int)x_rows; a.out_rows = (int)(r * top);
  a.parts = 1; a.kb_per_part = (int)(k / kBlock);
  a.ws_dtype = scale_dtype;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (contribution_dtype) {
    case AKAS_DTYPE_F32: launch_partial<AKAS_DTYPE_F32, kCombine>(a, s); break;
    case AKAS_DTYPE_BF16: launch_partial<AKAS_DTYPE_BF16, kCombine>(a, s); break;
    default: launch_partial<AKAS_DTYPE_F16, kCombine>(a, s);
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_fp8_expert_swiglu(const uint8_t* x, const float* activation_scales,
                                      const uint8_t* w, const void* w_scales, const uint8_t* w2,
                                      const void* w2_scales, int scale_dtype,
                                      const int32_t* counts, const int32_t* routes,
                                      const int32_t* tile_experts, const int32_t* tile_offsets,
                                      const int32_t* expert_offsets, uint8_t* out,
                                      float* output_scales, int64_t r, int top, int experts,
                                      int64_t o, int64_t k, int product_dtype,
                                      int activation_dtype, int max_block_m, int packed_input,
                                      int packed_output, void* stream) {
  (void)tile_experts;
  (void)tile_offsets;
  const int64_t x_rows =
      packed_input ? capacity_tiles(r, top, experts, max_block_m) * max_block_m : r;
  int st = check_common(r, top, experts, o, k, max_block_m, packed_input, x_rows);
  if (st != AKAS_OK) return st;
  if (packed_output && !packed_input) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(product_dtype) || !float_dtype(activation_dtype) || !scale_dtype_ok(scale_dtype))
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !activation_scales || !w || !w_scales || !w2 || !w2_scales || !counts || !routes ||
      !out || !output_scales)
    return AKAS_ERR_NULL;
  if ((packed_input || packed_output) && !expert_offsets) return AKAS_ERR_NULL;
  ExpertArgs a{};
  a.x = x; a.as = activation_scales; a.w = w; a.ws = w_scales; a.w2 = w2; a.ws2 = w2_scales;
  a.counts = counts; a.routes = routes; a.offsets = expert_offsets;
  a.out = out; a.out_scales = output_scales;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.routed = 0; a.packed_in = packed_input; a.packed_out = packed_output;
  a.x_rows = (int)x_rows;
  a.out_rows = (int)(packed_output ? capacity_tiles(r, top, experts, max_block_m) * max_block_m
                                   : r * top);
  a.parts = 1; a.kb_per_part = (int)(k / kBlock);
  a.ws_dtype = scale_dtype; a.prod_dtype = product_dtype; a.act_dtype = activation_dtype;
  launch_swiglu(a, reinterpret_cast<hipStream_t>(stream));
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_routed_fp8_expert_swiglu(
    const int32_t* ids, const int32_t* active, int32_t* counts, int32_t* routes, const uint8_t* x,
    const float* activation_scales, const uint8_t* w, const void* w_scales, const uint8_t* w2,
    const void* w2_scales, int scale_dtype, uint8_t* out, float* output_scales, int64_t r,
    int top, int experts, int64_t o, int64_t k, int product_dtype, int activation_dtype,
    void* stream) {
  int st = check_common(r, top, experts, o, k, 32, 0, r);
  if (st != AKAS_OK) return st;
  if (!float_dtype(product_dtype) || !float_dtype(activation_dtype) || !scale_dtype_ok(scale_dtype))
    return AKAS_ERR_DTYPE;
  if (!counts) return AKAS_ERR_NULL;
  if (r > 0 && (!ids || !routes || !x || !activation_scales || !w || !w_scales || !w2 ||
                !w2_scales || !out || !output_scales))
    return AKAS_ERR_NULL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ExpertArgs a{};
  a.x = x; a.as = activation_scales; a.w = w; a.ws = w_scales; a.w2 = w2; a.ws2 = w2_scales;
  a.counts = counts; a.routes = routes;
  a.ids = ids; a.active = active; a.scan_counts = counts; a.scan_routes = routes;
  a.scan_cols = top;
  a.out = out; a.out_scales = output_scales;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.x_rows = (int)r; a.out_rows = (int)(r * top);
  a.parts = 1; a.kb_per_part = (int)(k / kBlock);
  a.ws_dtype = scale_dtype; a.prod_dtype = product_dtype; a.act_dtype = activation_dtype;
  if (scan_fits(r, top, top, experts)) {
    launch_paired<kSwigluFp8, AKAS_DTYPE_F32, 1>(a, s);
  } else {
    launch_quantized_routes(ids, active, counts, routes, r, experts, top, s);
    if (r > 0) launch_swiglu(a, s);
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_expert_swiglu(const uint8_t* x, const float* activation_scales,
                                  const uint8_t* w, const void* w_scales, const uint8_t* w2,
                                  const void* w2_scales, int scale_dtype, const int32_t* counts,
                                  const int32_t* routes, const int32_t* tile_experts,
                                  const int32_t* tile_offsets, const int32_t* expert_offsets,
                                  void* out, int out_dtype, int64_t r, int top, int experts,
                                  int64_t o, int64_t k, int product_dtype, int activation_dtype,
                                  int max_block_m, int packed_input, int packed_output,
                                  void* stream) {
  (void)tile_experts;
  (void)tile_offsets;
  const int64_t x_rows =
      packed_input ? capacity_tiles(r, top, experts, max_block_m) * max_block_m : r;
  int st = check_common(r, top, experts, o, k, max_block_m, packed_input, x_rows);
  if (st != AKAS_OK) return st;
  if (packed_output && !packed_input) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(product_dtype) || !float_dtype(activation_dtype) || !float_dtype(out_dtype) ||
      !scale_dtype_ok(scale_dtype))
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !activation_scales || !w || !w_scales || !w2 || !w2_scales || !counts || !routes ||
      !out)
    return AKAS_ERR_NULL;
  if ((packed_input || packed_output) && !expert_offsets) return AKAS_ERR_NULL;
  ExpertArgs a{};
  a.x = x; a.as = activation_scales; a.w = w; a.ws = w_scales; a.w2 = w2; a.ws2 = w2_scales;
  a.counts = counts; a.routes = routes; a.offsets = expert_offsets; a.out = out;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.routed = 0; a.packed_in = packed_input; a.packed_out = packed_output;
  a.x_rows = (int)x_rows;
  a.out_rows = (int)(packed_output ? capacity_tiles(r, top, experts, max_block_m) * max_block_m
                                   : r * top);
  a.parts = 1; a.kb_per_part = (int)(k / kBlock);
  a.ws_dtype = scale_dtype; a.prod_dtype = product_dtype; a.act_dtype = activation_dtype;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case AKAS_DTYPE_F32: launch_paired<kSwiglu, AKAS_DTYPE_F32>(a, s); break;
    case AKAS_DTYPE_BF16: launch_paired<kSwiglu, AKAS_DTYPE_BF16>(a, s); break;
    default: launch_paired<kSwiglu, AKAS_DTYPE_F16>(a, s);
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_expert_pair_partial(const uint8_t* x, const float* activation_scales,
                                        const uint8_t* w, const void* w_scales, const uint8_t* w2,
                                        const void* w2_scales, int scale_dtype,
                                        const int32_t* counts, const int32_t* routes,
                                        const int32_t* tile_experts, const int32_t* tile_offsets,
                                        float* gate, float* up, int64_t r, int top, int experts,
                                        int64_t o, int64_t k, int partitions, int max_block_m,
                                        void* stream) {
  (void)tile_experts;
  (void)tile_offsets;
  int st = check_common(r, top, experts, o, k, max_block_m, 0, r);
  if (st != AKAS_OK) return st;
  if (partitions < 1 || (k / kBlock) % partitions) return AKAS_ERR_GEOMETRY;
  if (!scale_dtype_ok(scale_dtype)) return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !activation_scales || !w || !w_scales || !w2 || !w2_scales || !counts || !routes ||
      !gate || !up)
    return AKAS_ERR_NULL;
  ExpertArgs a{};
  a.x = x; a.as = activation_scales; a.w = w; a.ws = w_scales; a.w2 = w2; a.ws2 = w2_scales;
  a.counts = counts; a.routes = routes; a.out = gate; a.out2 = up;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.routed = 0; a.packed_in = 0; a.packed_out = 0;
  a.x_rows = (int)r; a.out_rows = (int)(r * top);
  a.parts = partitions; a.kb_per_part = (int)(k / kBlock / partitions);
  a.ws_dtype = scale_dtype;
  launch_paired<kPairPartial, AKAS_DTYPE_F32>(a, reinterpret_cast<hipStream_t>(stream));
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

// fp8_experts workspace: row-major codes and scales of the quantized input,
// then the per-expert counts and routes built from the group tables.
static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static int64_t fp8_experts_rows(int64_t r, int top, int routed_input) {
  return routed_input ? r * top : r;
}

extern "C" size_t akas_fp8_experts_workspace_size(int64_t r, int top, int experts, int64_t k,
                                                  int routed_input) {
  if (r <= 0 || top < 1 || experts < 1 || k <= 0) return 0;
  const int64_t rows = fp8_experts_rows(r, top, routed_input);
  return align256((size_t)(rows * k)) + align256((size_t)(rows * (k / kBlock)) * sizeof(float)) +
         align256((size_t)experts * sizeof(int32_t)) + (size_t)experts * (size_t)r * sizeof(int32_t);
}

extern "C" int akas_fp8_experts(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                                int scale_dtype, const int32_t* group_experts,
                                const int32_t* group_routes, void* out, int out_dtype,
                                void* workspace, size_t workspace_bytes, int64_t r, int top,
                                int experts, int64_t o, int64_t k, int routed_input,
                                void* stream) {
  const int64_t rows = r < 0 || top < 1 ? 0 : fp8_experts_rows(r, top, routed_input);
  int st = check_common(r, top, experts, o, k, 64, 0, rows);
  if (st != AKAS_OK) return st;
  if (r * top > 0x7FFFFFFF || (uint64_t)experts * (uint64_t)r >= (1ull << 31))
    return AKAS_ERR_GEOMETRY;
  if (!float_dtype(x_dtype) || !float_dtype(out_dtype) || !scale_dtype_ok(scale_dtype))
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !w || !w_scales || !group_experts || !group_routes || !out) return AKAS_ERR_NULL;
  if (!workspace || workspace_bytes < akas_fp8_experts_workspace_size(r, top, experts, k, routed_input))
    return AKAS_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint8_t* codes = reinterpret_cast<uint8_t*>(workspace);
  float* scales = reinterpret_cast<float*>(codes + align256((size_t)(rows * k)));
  int32_t* counts = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(scales) +
                                               align256((size_t)(rows * (k / kBlock)) * sizeof(float)));
  int32_t* routes = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(counts) +
                                               align256((size_t)experts * sizeof(int32_t)));
  st = launch_quantize(x, x_dtype, codes, scales, rows, k, false, s);
  if (st != AKAS_OK) return st;
  groups_to_routes_kernel<<<experts, 256, 0, s>>>(group_experts, group_routes, counts, routes, r,
                                                  top);
  ExpertArgs a{};
  a.x = codes; a.as = scales; a.w = w; a.ws = w_scales;
  a.counts = counts; a.routes = routes; a.out = out;
  a.r = (int)r; a.top = top; a.E = experts; a.N = (int)o; a.K = (int)k;
  a.routed = routed_input; a.packed_in = 0; a.packed_out = 0;
  a.x_rows = (int)rows; a.out_rows = (int)(r * top);
  a.parts = 1; a.kb_per_part = (int)(k / kBlock);
  a.ws_dtype = scale_dtype;
  switch (out_dtype) {
    case AKAS_DTYPE_F32: launch_partial<AKAS_DTYPE_F32>(a, s); break;
    case AKAS_DTYPE_BF16: launch_partial<AKAS_DTYPE_BF16>(a, s); break;
    default: launch_partial<AKAS_DTYPE_F16>(a, s);
  }
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

// ---------------------------------------------------------------------------
// The shared-expert MoE block in one call: the shared expert is expert E of
// the routed launches (rank `top` of every row), so the block is six
// launches (router, quantize, routes, gate/up + SwiGLU + requant, down,
// combine) with no dense launches beside them.
// ---------------------------------------------------------------------------
namespace {

struct BlockLayout {
  size_t ids, weights, codes, scales, counts, routes, act, act_scales, contributions, total;
};

BlockLayout block_layout(int64_t r, int experts, int top, int64_t h, int64_t f) {
  BlockLayout L{};
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += align256(bytes);
    return o;
  };
  const int64_t ranks = r * (top + 1);
  L.ids = take((size_t)(r * top) * sizeof(int32_t));
  L.weights = take((size_t)(r * top) * sizeof(float));
  L.codes = take((size_t)(r * h));
  L.scales = take((size_t)(r * (h / kBlock)) * sizeof(float));
  L.counts = take((size_t)(experts + 1) * sizeof(int32_t));
  L.routes = take((size_t)(experts + 1) * (size_t)r * sizeof(int32_t));
  L.act = take((size_t)(ranks * f));
  L.act_scales = take((size_t)(ranks * (f / kBlock)) * sizeof(float));
  L.contributions = take((size_t)(ranks * h) * sizeof(uint16_t));
  L.total = at;
  return L;
}

}  // namespace

extern "C" size_t akas_shared_expert_moe_workspace_size(int64_t r, int experts, int top, int64_t h,
                                                        int64_t f) {
  if (r <= 0 || experts < 1 || top < 1 || h <= 0 || f <= 0) return 0;
  return block_layout(r, experts, top, h, f).total;
}

extern "C" int akas_shared_expert_moe(
    const void* x, int x_dtype, const float* logits, const void* shared_gate, int gate_dtype,
    const uint8_t* w1, const void* s1, const uint8_t* w3, const void* s3, const uint8_t* w2,
    const void* s2, const uint8_t* sw1, const void* ss1, const uint8_t* sw3, const void* ss3,
    const uint8_t* sw2, const void* ss2, int scale_dtype, float* out, void* workspace,
    size_t workspace_bytes, int64_t r, int experts, int top, int64_t h, int64_t f,
    void* stream) {
  if (r < 0 || experts < 1 || experts + 1 > 1024 || top < 1 || top > 32 || top > experts ||
      h <= 0 || f <= 0 || h % kBlock || f % kBlock || r > 65535 * 64)
    return AKAS_ERR_GEOMETRY;
  const int64_t ranks = r * (top + 1);
  int st = check_common(r, top + 1, experts + 1, f, h, 64, 0, r);
  if (st == AKAS_OK) st = check_common(r, top + 1, experts + 1, h, f, 64, 0, ranks);
  if (st != AKAS_OK) return st;
  if ((uint64_t)(experts + 1) * (uint64_t)r >= (1ull << 31)) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(x_dtype) || !float_dtype(gate_dtype) || !scale_dtype_ok(scale_dtype))
    return AKAS_ERR_DTYPE;
  if (r == 0) return AKAS_OK;
  if (!x || !logits || !shared_gate || !w1 || !s1 || !w3 || !s3 || !w2 || !s2 || !sw1 || !ss1 ||
      !sw3 || !ss3 || !sw2 || !ss2 || !out)
    return AKAS_ERR_NULL;
  const BlockLayout L = block_layout(r, experts, top, h, f);
  if (!workspace || workspace_bytes < L.total) return AKAS_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return AKAS_ERR_GEOMETRY;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint8_t* base = reinterpret_cast<uint8_t*>(workspace);
  int32_t* ids = reinterpret_cast<int32_t*>(base + L.ids);
  float* weights = reinterpret_cast<float*>(base + L.weights);
  uint8_t* codes = base + L.codes;
  float* scales = reinterpret_cast<float*>(base + L.scales);
  int32_t* counts = reinterpret_cast<int32_t*>(base + L.counts);
  int32_t* routes = reinterpret_cast<int32_t*>(base + L.routes);
  uint8_t* act = base + L.act;
  float* act_scales = reinterpret_cast<float*>(base + L.act_scales);
  uint16_t* contributions = reinterpret_cast<uint16_t*>(base + L.contributions);

  st = launch_decode_router_quantize(logits, ids, weights, r, experts, top, x, x_dtype, codes,
                                     scales, h, s);
  if (st != AKAS_OK) return st;
  ExpertArgs g{};
  g.x = codes; g.as = scales; g.w = w1; g.ws = s1; g.w2 = w3; g.ws2 = s3;
  g.xw = sw1; g.xws = ss1; g.xw2 = sw3; g.xws2 = ss3;
  g.counts = counts; g.routes = routes; g.out = act; g.out_scales = act_scales;
  g.r = (int)r; g.top = top + 1; g.E = experts + 1; g.N = (int)f; g.K = (int)h;
  g.x_rows = (int)r; g.out_rows = (int)ranks;
  g.parts = 1; g.kb_per_part = (int)(h / kBlock);
  g.ws_dtype = scale_dtype; g.prod_dtype = AKAS_DTYPE_F32; g.act_dtype = AKAS_DTYPE_F32;
  // Decode batches scan the routes inside the gate/up launch (counts and
  // routes as launch_routes_with_shared leaves them); larger ones take the
  // route scan's own launch.
  if (scan_fits(r, top, top + 1, experts + 1)) {
    g.ids = ids; g.scan_counts = counts; g.scan_routes = routes; g.scan_cols = top;
    launch_paired<kSwigluFp8, AKAS_DTYPE_F32, 1>(g, s);
  } else {
    launch_routes_with_shared(ids, counts, routes, r, experts, top, s);
    launch_swiglu(g, s);
  }

  ExpertArgs d{};
  d.x = act; d.as = act_scales; d.w = w2; d.ws = s2; d.xw = sw2; d.xws = ss2;
  d.counts = counts; d.routes = routes; d.out = contributions;
  d.r = (int)r; d.top = top + 1; d.E = experts + 1; d.N = (int)h; d.K = (int)f;
  d.routed = 1; d.x_rows = (int)ranks; d.out_rows = (int)ranks;
  d.parts = 1; d.kb_per_part = (int)(f / kBlock);
  d.ws_dtype = scale_dtype;
  launch_partial<AKAS_DTYPE_BF16>(d, s);

  launch_shared_rank_combine(contributions, weights, shared_gate, gate_dtype, out, r, top, h, s);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}
