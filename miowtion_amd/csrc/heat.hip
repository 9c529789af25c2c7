// Teacher block heat for gfx950: per (head, query tile, key tile) the block's
// softmax mass ('sum') or peak probability ('max') from the dense LSE.
//
// Workgroup = (head, group of four query items): 16 waves walk every key tile
// of the head once, so each K tile fetched into LDS serves four query tiles.
// Wave w owns query item w / 4 of the group and its rows 32 (w % 4) .. + 31,
// and all 64 keys of every step (two 32-key sub-blocks). Steps are 64-key halves of
// the key tiles in tile order (a tile's halves consecutive; rows past its
// valid count not fetched, an empty half no step), through a 4-slot LDS ring
// with three steps in flight. Each wave keeps its rows' Q^T in registers as
// the B operand of S^T = K Q^T (v_mfma_f32_32x32x16_bf16), so a lane holds
// one query row and 16 keys of a sub-block; a lane accumulates its share of
// the current key tile in a register and the wave reduces it (DPP and lane
// swaps) once, at the tile's last step, into an LDS table (two of them,
// alternating); after the next barrier the first wave of each item adds the
// item's four entries in a fixed order into the item's slot for the tile, so
// the result does not depend on timing. Only one fp32 value per block
// leaves the workgroup.

#include "veda_common.h"
#include "veda_pipeline.h"

namespace veda {
namespace {

constexpr int kD = 128;
constexpr int kHeatThreads = 1024;
constexpr int kHeatItems = 4;  // query items per workgroup
constexpr int kMaxTiles = 2048;  // key tiles per layout (FA4's block-mask cap)
constexpr float kLog2e = 1.4426950408889634f;

struct HeatParams {
  const uint16_t* q;
  const uint16_t* k;
  int64_t qs, qh, ks, kh;
  const float* lse;
  int64_t ls, lh;
  const int32_t* valid_count;
  const int64_t* q_tiles;
  int64_t n_q, n_tiles, n_heads;
  float scale;
  float* heat;
};

// Per-lane byte offsets of this wave's 1 KB K segment of a step (segment =
// wave: rows 4 wave + l / 16, LDS chunk l % 16 holding logical chunk
// (l % 16) ^ (row & 15)) and of its redirect (rows l / 16) for a segment
// wholly past the valid count.
struct KDma {
  uint32_t k, skip;
};

__device__ __forceinline__ KDma kdma_offsets(int64_t ks, int wave, int lane) {
  const int lr = lane >> 4, pc = lane & 15;
  const int row = 4 * wave + lr;
  const int kc = (pc ^ (row & 15)) << 3;
  return KDma{(uint32_t)((row * ks + kc) * 2), (uint32_t)((lr * ks + kc) * 2)};
}

template <int REDUCE>  // 0: sum, 1: max
__global__ void __launch_bounds__(kHeatThreads) heat_kernel(HeatParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t kr0[kHalfBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t kr1[kHalfBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t kr2[kHalfBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t kr3[kHalfBytes];
  __shared__ uint16_t steps[2 * kMaxTiles];  // (key tile << 2) | (half << 1) | last of tile
  __shared__ uint8_t tvc[kMaxTiles];
  __shared__ float part[kHeatItems][kMaxTiles];
  __shared__ float tilebuf[2][16];  // per wave, a key tile's reduced share; two tables, alternating
  __shared__ int32_t step_total;
  lds_u8* K0 = (lds_u8*)kr0;
  lds_u8* K1 = (lds_u8*)kr1;
  lds_u8* K2 = (lds_u8*)kr2;
  lds_u8* K3 = (lds_u8*)kr3;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int pick = wave >> 2, rg = wave & 3;  // item of the pair, row group
  const int li = lane & 31, hi = lane >> 5;
  const int64_t n_groups = (p.n_q + kHeatItems - 1) / kHeatItems;
  const int64_t head = blockIdx.x / n_groups;
  const int64_t r = (blockIdx.x % n_groups) * kHeatItems + pick;
  const int nt = (int)p.n_tiles;
  const bool item_ok = r < p.n_q;
  const int64_t qt = item_ok ? p.q_tiles[r] : -1;
  const bool qt_ok = qt >= 0 && qt < p.n_tiles;

  // Partials start empty (a tile no step reaches keeps them); the step
  // list is built by wave 0: every tile with a valid key, its first half and
  // then its second half when more than 64 keys are valid, in tile order
  // (positions from a ballot prefix).
  for (int j = tid; j < nt; j += kHeatThreads) {
    tvc[j] = (uint8_t)min(max(p.valid_count[j], 0), kTile);
#pragma unroll
    for (int it = 0; it < kHeatItems; ++it) part[it][j] = REDUCE ? -INFINITY : 0.f;
  }
  if (wave == 0) {
    int n = 0;
    for (int j0 = 0; j0 < nt; j0 += 64) {
      const int j = j0 + lane;
      const int vc = j < nt ? min(max(p.valid_count[j], 0), kTile) : 0;
      const bool one = vc > 0, two = vc > kHalf;
      const uint64_t b1 = __ballot(one), b2 = __ballot(two);
      const int rank =
          __builtin_amdgcn_mbcnt_hi((uint32_t)(b1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b1, 0)) +
          __builtin_amdgcn_mbcnt_hi((uint32_t)(b2 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b2, 0));
      if (one) steps[n + rank] = (uint16_t)((j << 2) | (two ? 0 : 1));
      if (two) steps[n + rank + 1] = (uint16_t)((j << 2) | 2 | 1);
      n += __builtin_popcountll(b1) + __builtin_popcountll(b2);
    }
    if (lane == 0) step_total = n;
  }

  const int vcq = qt_ok ? min(max(p.valid_count[qt], 0), kTile) : 0;
  const int row = 32 * rg + li;
  const bool row_ok = row < vcq;
  const int64_t qrow = (qt_ok ? qt : 0) * kTile + row;
  bf16x8 qf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const u32x4 v = row_ok ? ld16(p.q + qrow * p.qs + head * p.qh + 16 * s + 8 * hi)
                           : u32x4{0, 0, 0, 0};
    qf[s] = __builtin_bit_cast(bf16x8, v);
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" : : "v"(qf[s]));
  const float lse = row_ok ? p.lse[qrow * p.ls + head * p.lh] : 0.f;
  // sum: exp2(s * c2 - lse2); an invalid row has lse2 = +inf (adds 0).
  const float c2 = p.scale * kLog2e;
  const float lse2 = row_ok ? lse * kLog2e : INFINITY;
  __syncthreads();  // partials, valid counts and step list ready
  const int n_steps = __builtin_amdgcn_readfirstlane(step_total);

  uint32_t kfo[8];  // K fragment offsets: row li (+ 32 sub-block), logical chunk 2s + hi
  {
    const uint32_t krow = li * 256, x = (hi ^ (li & 15)) << 4;
#pragma unroll
    for (int s = 0; s < 8; ++s) kfo[s] = krow + (x ^ (s << 5));
  }
  const KDma dma = kdma_offsets(p.ks, wave, lane);
  const uint16_t* kbase = p.k + head * p.kh;
  auto entry = [&](int u) { return __builtin_amdgcn_readfirstlane((int)steps[u]); };
  auto valid_of = [&](int e) {  // valid keys of the step's half
    const int vc = __builtin_amdgcn_readfirstlane((int)tvc[e >> 2]);
    return (e & 2) ? vc - kHalf : min(vc, kHalf);
  };
  auto load_step = [&](int u, lds_u8* slot) {
    const int e = entry(u);
    const int64_t row0 = (int64_t)(e >> 2) * kTile + ((e >> 1) & 1) * kHalf;
    const int vch = valid_of(e);
    const char* b = reinterpret_cast<const char*>(kbase + row0 * p.ks);
    dma16(b, 4 * wave < vch ? dma.k : dma.skip, slot + wave * 1024);
  };
  float acc = REDUCE ? -INFINITY : 0.f;  // this lane's share of the current key tile
  // (wave-uniform) key tile whose table entries wait for the combine, the
  // table they are in, and the number of tiles ended so far
  int pend = -1, pend_tab = 0, ends = 0;
  auto combine = [&]() {
    if (pend >= 0 && rg == 0 && lane == 0) {
      const float* t = tilebuf[pend_tab] + 4 * pick;
      float v = t[0];
#pragma unroll
      for (int w = 1; w < 4; ++w) v = REDUCE ? fmaxf(v, t[w]) : v + t[w];
      part[pick][pend] = v;
    }
    pend = -1;
  };
  // One 32-key sub-block (keys kb .. kb + 31 of the half, lim of them valid).
  auto sub_block = [&](const lds_u8* slot, int kb, int lim) {
    u32x4 kf[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      kf[s] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(slot + kb * 256 + kfo[s]);
    f32x16 sacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kf[s]), qf[s],
                                                     sacc, 0, 0, 0);
    // Register e holds key kb + 8 (e / 4) + 4 hi + e % 4 of the half.
    if (lim < 32) {
      const int l = lim - 4 * hi;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (8 * (e >> 2) + (e & 3) >= l) sacc[e] = -INFINITY;
    }
    if (REDUCE) {
#pragma unroll
      for (int e = 0; e < 16; ++e) acc = fmaxf(acc, sacc[e]);
    } else {
      float a[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        a[g] = 0.f;
#pragma unroll
        for (int m = 0; m < 4; ++m) a[g] += __builtin_amdgcn_exp2f(fmaf(sacc[4 * g + m], c2, -lse2));
      }
      acc += (a[0] + a[1]) + (a[2] + a[3]);
    }
  };
  auto compute_step = [&](int u, const lds_u8* slot) {
    combine();  // the previous tile's entries are visible after this step's barrier
    const int e = entry(u);
    const int vch = valid_of(e);
    sub_block(slot, 0, vch);
    if (vch > 32) sub_block(slot, 32, vch - 32);
    if (e & 1) {  // the tile's last step: reduce over the wave into its slot
      float v;
      if (REDUCE) {
        // Row max over the tile's keys, rounded to bf16 like the
        // reference's bf16 scores (rounding is monotonic, so rounding the
        // max is rounding every score), then max over rows of
        // max * scale - lse.
        float rm = half_swap_max(acc);
        if (rm != -INFINITY) rm = bf16_to_f32(f32_to_bf16(rm));
        v = (rm == -INFINITY || !row_ok) ? -INFINITY : rm * p.scale - lse;
        v = wave_reduce<true>(v);
      } else {
        v = wave_reduce<false>(acc);
      }
      // consecutive tile ends alternate tables, so a table is written again
      // only after the barrier that follows its combine
      pend_tab = ends & 1;
      ++ends;
      if (lane == 0) tilebuf[pend_tab][wave] = v;
      pend = e >> 2;
      acc = REDUCE ? -INFINITY : 0.f;
    }
  };
  // The ring: step u in slot u & 3; at the top of step u its own load is
  // waited for (those of u+1, u+2 may stay in flight) together with this
  // wave's LDS stores (the tile table), then a bare barrier (as in the
  // attention kernel), then the slot step u-1 used is refilled with step
  // u+3. Every row of a slot that a step reads was written by that step's
  // loads (segments past the valid count re-read real rows).
  auto top = [&](int u) {
    // s_waitcnt vmcnt(n) lgkmcnt(0)
    if (u + 2 < n_steps) __builtin_amdgcn_s_waitcnt(0x0070 | 2);
    else if (u + 1 < n_steps) __builtin_amdgcn_s_waitcnt(0x0070 | 1);
    else __builtin_amdgcn_s_waitcnt(0x0070);
    __builtin_amdgcn_s_barrier();
  };
  if (n_steps > 0) load_step(0, K0);
  if (n_steps > 1) load_step(1, K1);
  if (n_steps > 2) load_step(2, K2);
  for (int u = 0; u < n_steps; u += 4) {
    top(u);
    if (u + 3 < n_steps) load_step(u + 3, K3);
    compute_step(u, K0);
    if (u + 1 >= n_steps) break;
    top(u + 1);
    if (u + 4 < n_steps) load_step(u + 4, K0);
    compute_step(u + 1, K1);
    if (u + 2 >= n_steps) break;
    top(u + 2);
    if (u + 5 < n_steps) load_step(u + 5, K1);
    compute_step(u + 2, K2);
    if (u + 3 >= n_steps) break;
    top(u + 3);
    if (u + 6 < n_steps) load_step(u + 6, K2);
    compute_step(u + 3, K3);
  }
  __syncthreads();  // the last tile's table entries written
  combine();
  __syncthreads();  // all partials written
#pragma unroll
  for (int it = 0; it < kHeatItems; ++it) {
    const int64_t rr = (blockIdx.x % n_groups) * kHeatItems + it;
    if (rr >= p.n_q) break;
    const int64_t qti = p.q_tiles[rr];
    const bool ok = qti >= 0 && qti < p.n_tiles;  // not a query tile of this layout: no heat
    float* heat_row = p.heat + (head * p.n_q + rr) * p.n_tiles;
    for (int j = tid; j < nt; j += kHeatThreads) {
      float v = part[it][j];
      if (REDUCE) v = v == -INFINITY ? 0.f : expf(v);
      heat_row[j] = ok ? v : 0.f;
    }
  }
}

// Heat from the block statistics of the teacher's dense pass in tile order
// (veda_dense_heat_fwd): part[h][j][row] is the log2 log-sum-exp ('sum') or
// log2 max ('max') of query row `row` over the valid keys of key tile j,
// lse[h][row] the row's natural-log LSE over all keys. Then
//   'sum': heat[h, r, j] = sum over valid rows of 2^(part - lse log2 e)
//   'max': heat[h, r, j] = 2^(max over valid rows of (part - lse log2 e))
// (0 when nothing is valid), the block's softmax mass / peak probability.
// Workgroup = (head, query item), 4 waves; wave w takes key tiles w, w + 4,
// ..., each a 512-byte coalesced read of the item's 128 rows.
template <bool REDUCE>
__global__ void __launch_bounds__(256) heat_combine_kernel(
    const float* __restrict__ part, const float* __restrict__ lse, int64_t ls_h, int64_t ls_s,
    const int32_t* __restrict__ valid_count, const int64_t* __restrict__ q_tiles,
    int64_t n_items, int64_t n_tiles, float* __restrict__ heat) {
  const int64_t item = blockIdx.x;
  const int64_t h = item / n_items, r = item % n_items;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t qt = q_tiles != nullptr ? q_tiles[r] : r;
  const int vc = (qt >= 0 && qt < n_tiles) ? valid_count[qt] : 0;
  float l2[2];
  bool ok[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int slot = lane + 64 * x;
    const float l = lse[h * ls_h + (r * kTile + slot) * ls_s];
    ok[x] = slot < vc && l != -INFINITY;
    l2[x] = l * kLog2e;
  }
  const int64_t rows = n_items * kTile;
  const float* base = part + h * n_tiles * rows + r * kTile;
  float* out = heat + (h * n_items + r) * n_tiles;
  for (int64_t j = wave; j < n_tiles; j += 4) {
    const float* pr = base + j * rows;
    const float x0 = pr[lane], x1 = pr[lane + 64];
    float v;
    if (REDUCE) {
      v = fmaxf(ok[0] ? x0 - l2[0] : -INFINITY, ok[1] ? x1 - l2[1] : -INFINITY);
      v = wave_reduce<true>(v);
      v = v == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(v);
    } else {
      v = (ok[0] ? __builtin_amdgcn_exp2f(x0 - l2[0]) : 0.f) +
          (ok[1] ? __builtin_amdgcn_exp2f(x1 - l2[1]) : 0.f);
      v = wave_reduce<false>(v);
    }
    if (lane == 0) out[j] = v;
  }
}

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" int veda_block_heat(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                               const void* k, int64_t k_stride_s, int64_t k_stride_h,
                               const float* lse, int64_t lse_stride_s, int64_t lse_stride_h,
                               const int32_t* valid_count, const int64_t* q_tiles, int64_t n_q,
                               int64_t n_tiles, int64_t n_heads, int64_t head_dim, int reduce,
                               float scale, float* heat, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_heat: head_dim must be 128, got %lld", (long long)head_dim);
  VEDA_REQUIRE(reduce == 0 || reduce == 1, "block_heat: reduce must be 0 (sum) or 1 (max)");
  VEDA_REQUIRE(q_stride_s % 8 == 0 && q_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   k_stride_h % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(k) & 15) == 0,
               "block_heat: rows must be 16-byte aligned");
  VEDA_REQUIRE(n_q >= 0 && n_tiles >= 0 && n_heads >= 0, "block_heat: negative size");
  VEDA_REQUIRE(n_tiles <= kMaxTiles, "block_heat: %lld key tiles, at most %d",
               (long long)n_tiles, kMaxTiles);
  if (n_q == 0 || n_tiles == 0 || n_heads == 0) return VEDA_OK;
  HeatParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.qs = q_stride_s; p.qh = q_stride_h; p.ks = k_stride_s; p.kh = k_stride_h;
  p.lse = lse; p.ls = lse_stride_s; p.lh = lse_stride_h;
  p.valid_count = valid_count; p.q_tiles = q_tiles;
  p.n_q = n_q; p.n_tiles = n_tiles; p.n_heads = n_heads;
  p.scale = scale; p.heat = heat;
  const int64_t items = n_heads * ((n_q + kHeatItems - 1) / kHeatItems);  // per group of items
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (reduce) heat_kernel<1><<<(unsigned)items, kHeatThreads, 0, s>>>(p);
  else heat_kernel<0><<<(unsigned)items, kHeatThreads, 0, s>>>(p);
  return check_launch("veda_block_heat");
}

extern "C" int veda_heat_combine(const float* part, const float* lse, int64_t lse_stride_h,
                                 int64_t lse_stride_s, const int32_t* valid_count,
                                 const int64_t* q_tiles, int64_t n_items, int64_t n_tiles,
                                 int64_t n_heads, int reduce, float* heat, void* stream) {
  VEDA_REQUIRE(reduce == 0 || reduce == 1, "heat_combine: reduce must be 0 (sum) or 1 (max)");
  VEDA_REQUIRE(n_items >= 0 && n_tiles >= 0 && n_heads >= 0, "heat_combine: negative size");
  if (n_items == 0 || n_tiles == 0 || n_heads == 0) return VEDA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned g = (unsigned)(n_heads * n_items);
  if (reduce)
    heat_combine_kernel<true><<<g, 256, 0, s>>>(part, lse, lse_stride_h, lse_stride_s, valid_count,
                                                q_tiles, n_items, n_tiles, heat);
  else
    heat_combine_kernel<false><<<g, 256, 0, s>>>(part, lse, lse_stride_h, lse_stride_s,
                                                 valid_count, q_tiles, n_items, n_tiles, heat);
  return check_launch("veda_heat_combine");
}
