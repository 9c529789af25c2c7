// Block selection: equal-budget top-k per query tile, the block mask, and
// the full / partial key-tile lists the attention kernel walks.
//
// Top-k: one wave per (head, query tile). Scores become 64-bit keys
// (orderable fp32 score << 32 | ~column); lane l holds the keys of columns
// l, l + 64, .., sorts them in registers (a bitonic network over N = 16 or
// 32 keys, zeros padding the list) and keeps them in LDS in that order,
// lane-strided so every LDS access is conflict-free. k_hi rounds of a
// wave-wide max over the lanes' current heads extract the winners in
// descending order; the winning lane's next head is one LDS read. The
// rounds are a latency chain, so occupancy is what the kernel runs on: the
// LDS holds only the row's columns (dynamic size, 20 KB per workgroup at
// 592 columns: 8 workgroups per CU instead of the 2 a 2048-column array
// allows). Folding the column into the key makes every key distinct, so the
// order is total: higher score first, lower column first on equal scores.
//
// Lists: one wave per (head, row), 64 columns per step, positions from a
// ballot + popcount prefix (no sort, no atomics).

#include <type_traits>

#include "veda_common.h"

namespace veda {
namespace {

// Order key of a score: unsigned order of keys = numeric order of scores,
// with every NaN (either sign) one key above +inf, as torch.sort / topk rank
// NaN above every number (so NaNs tie among themselves and fall back to
// column order).
constexpr uint32_t kNaNKey = 0xffffffffu;
constexpr uint32_t kNegInfKey = 0x007fffffu;  // orderable(-inf)

__device__ __forceinline__ uint32_t orderable(float v) {
  if (v != v) return kNaNKey;
  if (v == 0.f) v = 0.f;  // -0 ties with +0, as in a float comparison
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_update_dpp(0u, (uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0u, (uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Max over the 64 lanes, wave-uniform. Within a 16-lane row: DPP exchanges
// with lane ^ 1, lane ^ 2, the mirror inside 8 and the mirror inside 16;
// across rows: a swizzle with lane ^ 16, then v_permlane32_swap with the
// lane 32 positions away (it leaves {own, partner} in its two results, in
// the same order for both halves of the key).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_u64(v, dpp_u64<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max_u64(v, dpp_u64<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max_u64(v, dpp_u64<0x141>(v));  // row_half_mirror
  v = max_u64(v, dpp_u64<0x140>(v));  // row_mirror
  {
    const uint32_t lo = __builtin_amdgcn_ds_swizzle((uint32_t)v, 0x401F);
    const uint32_t hi = __builtin_amdgcn_ds_swizzle((uint32_t)(v >> 32), 0x401F);
    v = max_u64(v, ((uint64_t)hi << 32) | lo);
  }
  const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32),
                                                   false, false);
  v = max_u64(((uint64_t)hi[0] << 32) | lo[0], ((uint64_t)hi[1] << 32) | lo[1]);
  const uint32_t ulo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t uhi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)uhi << 32) | ulo;
}

constexpr int kMaxCols = 2048;  // columns of one block (FA4's 2048-block cap)
constexpr int kSelWaves = 4;

// Sorts N keys descending (bitonic network, indices fixed at compile time,
// so the keys stay in registers).
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&k)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const uint64_t a = k[i], b = k[j];
          const bool sw = (i & size) == 0 ? a < b : a > b;
          k[i] = sw ? b : a;
          k[j] = sw ? a : b;
        }
      }
}

template <int N>  // keys per lane the registers hold (>= the row's columns / 64)
__global__ void __launch_bounds__(256) select_topk_kernel(
    const float* __restrict__ scores, int64_t n_heads, int64_t n_rows, int64_t ssh,
    int64_t ssr, int64_t block_start, int n_cols, const uint8_t* __restrict__ kv_ok,
    const int64_t* __restrict__ rows, int k_lo, int k_hi, const uint8_t* __restrict__ extra,
    int64_t n_extra, int64_t* __restrict__ index, uint8_t* __restrict__ keep, int64_t osh,
    int64_t osr, int64_t col0) {
  extern __shared__ uint64_t keys[];  // [kSelWaves][per_lane * 64]
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kSelWaves + wave;
  if (item >= n_heads * n_rows) return;  // whole wave exits together
  const int64_t h = item / n_rows, r = item % n_rows;
  const int64_t tile_id = rows[r];
  const int64_t diag = tile_id - block_start;  // column of the own tile, if in block
  const float* srow = scores + h * ssh + r * ssr + block_start;
  const int per_lane = (n_cols + 63) / 64;
  uint64_t* kv = keys + wave * per_lane * 64;
  uint64_t k[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int c = j * 64 + lane;
    uint64_t key = 0;  // absent column: below every real key
    if (j < per_lane && c < n_cols) {
      float v = srow[c];
      if (!kv_ok[block_start + c]) v = -INFINITY;
      if (c == diag) v = INFINITY;
      key = ((uint64_t)orderable(v) << 32) | (uint32_t)(~(uint32_t)c);
    }
    k[j] = key;
  }
  sort_desc(k);
#pragma unroll
  for (int j = 0; j < N; ++j)
    if (j < per_lane) kv[j * 64 + lane] = k[j];
  uint64_t best = k[0];
  int pos = 0;  // index of this lane's current head in its sorted list
  const bool has_extra = tile_id >= 0 && tile_id < n_extra && extra[tile_id] != 0;
  const int allowed = k_lo + (has_extra ? 1 : 0);
  int64_t* irow = index + h * osh + r * osr + col0;
  uint8_t* krow = keep + h * osh + r * osr + col0;
  for (int t = 0; t < k_hi; ++t) {
    const uint64_t top = wave_max_u64(best);
    const uint32_t c = ~(uint32_t)top;
    const uint32_t vkey = (uint32_t)(top >> 32);
    if ((int)(c & 63) == lane) {
      irow[t] = block_start + (int64_t)c;
      // kept: within the row's budget and `val > -inf` (False for NaN,
      // mask.py:251-284)
      krow[t] = (t < allowed && vkey > kNegInfKey && vkey != kNaNKey) ? 1 : 0;
      ++pos;
      best = pos < per_lane ? kv[pos * 64 + lane] : 0;
    }
  }
}

constexpr int kMaxTiles = 8192;

__global__ void __launch_bounds__(256) dense_mask_kernel(
    const int64_t* __restrict__ index, const uint8_t* __restrict__ keep, int64_t n_sel,
    int64_t k_total, const uint8_t* __restrict__ kv_ok, int n_tiles, int64_t n_video,
    int64_t out_rows, uint8_t* __restrict__ mask) {
  __shared__ uint8_t row[kMaxTiles];
  const int64_t h = blockIdx.x / out_rows, r = blockIdx.x % out_rows;
  const bool video_row = r < n_sel && r < n_video;
  for (int c = threadIdx.x; c < n_tiles; c += blockDim.x)
    row[c] = (!video_row || c >= n_video) ? kv_ok[c] : 0;
  __syncthreads();
  if (video_row) {
    const int64_t base = (h * n_sel + r) * k_total;
    for (int64_t t = threadIdx.x; t < k_total; t += blockDim.x) {
      const int64_t c = index[base + t];
      if (keep[base + t] && c >= 0 && c < n_tiles) row[c] = 1;
    }
  }
  __syncthreads();
  uint8_t* out = mask + (h * out_rows + r) * n_tiles;
  for (int c = threadIdx.x; c < n_tiles; c += blockDim.x) out[c] = row[c];
}

// Index lists: one wave per (head, row). The row's classes (0 outside the
// row's members, 1 full member, 2 partial member) are first staged in LDS
// with wide independent loads; the lists are then written 64 columns at a
// time, each lane storing its column once per list (members at their rank,
// non-members after all members), so every store instruction is whole.
// Rows longer than kListCols take the two-pass form from global memory.
constexpr int kListWaves = 4;
constexpr int kListCols = 4096;

template <int VEC>
__device__ __forceinline__ void stage_classes(const uint8_t* __restrict__ m,
                                              const uint8_t* __restrict__ kv_ok,
                                              const uint8_t* __restrict__ full_tile, int n_tiles,
                                              int lane, uint8_t* cls, int& counts) {
  using Vec = typename std::conditional<VEC == 16, uint4,
              typename std::conditional<VEC == 4, uint32_t, uint8_t>::type>::type;
  int nf = 0, np = 0;
#pragma unroll 4
  for (int c = lane * VEC; c < n_tiles; c += 64 * VEC) {
    union { Vec v; uint8_t b[VEC]; } mm, kk, ff, out;
    mm.v = *reinterpret_cast<const Vec*>(m + c);
    kk.v = *reinterpret_cast<const Vec*>(kv_ok + c);
    ff.v = *reinterpret_cast<const Vec*>(full_tile + c);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const bool member = mm.b[j] && kk.b[j];
      const bool full = ff.b[j] != 0;
      out.b[j] = member ? (full ? 1 : 2) : 0;
      nf += member && full;
      np += member && !full;
    }
    *reinterpret_cast<Vec*>(cls + c) = out.v;
  }
  counts = nf | (np << 16);  // both at most 4096
}

__global__ void __launch_bounds__(64 * kListWaves) index_lists_kernel(
    const uint8_t* __restrict__ mask, int64_t n_items, int n_tiles, int vec,
    const uint8_t* __restrict__ kv_ok, const uint8_t* __restrict__ full_tile,
    int32_t* __restrict__ part_cnt, int32_t* __restrict__ part_idx,
    int32_t* __restrict__ full_cnt, int32_t* __restrict__ full_idx) {
  __shared__ __align__(16) uint8_t cls_lds[kListWaves][kListCols];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kListWaves + wave;
  if (item >= n_items) return;  // each wave uses only its own LDS row
  const uint8_t* m = mask + item * n_tiles;
  int32_t* fi = full_idx + item * n_tiles;
  int32_t* pi = part_idx + item * n_tiles;
  const uint64_t below = (1ull << lane) - 1ull;
  if (n_tiles <= kListCols) {
    uint8_t* cls = cls_lds[wave];
    int counts;
    if (vec == 16)
      stage_classes<16>(m, kv_ok, full_tile, n_tiles, lane, cls, counts);
    else if (vec == 4)
      stage_classes<4>(m, kv_ok, full_tile, n_tiles, lane, cls, counts);
    else
      stage_classes<1>(m, kv_ok, full_tile, n_tiles, lane, cls, counts);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) counts += __shfl_xor(counts, off);
    const int NF = counts & 0xffff, NP = counts >> 16;
    // the lanes' LDS stores are seen by the other lanes of this wave
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int nf = 0, np = 0;  // members before the chunk
    for (int c0 = 0; c0 < n_tiles; c0 += 64) {
      const int c = c0 + lane;
      const int k = c < n_tiles ? cls[c] : 0;
      const uint64_t bf = __ballot(k == 1), bp = __ballot(k == 2);
      const int rf = __popcll(bf & below), rp = __popcll(bp & below);
      if (c < n_tiles) {
        fi[k == 1 ? nf + rf : NF + (c0 - nf) + (lane - rf)] = c;
        pi[k == 2 ? np + rp : NP + (c0 - np) + (lane - rp)] = c;
      }
      nf += __popcll(bf);
      np += __popcll(bp);
    }
    if (lane == 0) {
      full_cnt[item] = NF;
      part_cnt[item] = NP;
    }
    return;
  }
  int nf = 0, np = 0;
  for (int c0 = 0; c0 < n_tiles; c0 += 64) {
    const int c = c0 + lane;
    bool f = false, p = false;
    if (c < n_tiles && m[c] && kv_ok[c]) {
      f = full_tile[c] != 0;
      p = !f;
    }
    const uint64_t bf = __ballot(f), bp = __ballot(p);
    if (f) fi[nf + __popcll(bf & below)] = c;
    if (p) pi[np + __popcll(bp & below)] = c;
    nf += __popcll(bf);
    np += __popcll(bp);
  }
  // Non-members follow, ascending (the stable argsort of ~member).
  int of = nf, op = np;
  for (int c0 = 0; c0 < n_tiles; c0 += 64) {
    const int c = c0 + lane;
    bool f = false, p = false;
    if (c < n_tiles) {
      const bool member = m[c] && kv_ok[c];
      const bool full = full_tile[c] != 0;
      f = !(member && full);
      p = !(member && !full);
    }
    const uint64_t bf = __ballot(f), bp = __ballot(p);
    if (f) fi[of + __popcll(bf & below)] = c;
    if (p) pi[op + __popcll(bp & below)] = c;
    of += __popcll(bf);
    op += __popcll(bp);
  }
  if (lane == 0) {
    full_cnt[item] = nf;
    part_cnt[item] = np;
  }
}

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" int veda_select_topk(const float* scores, int64_t n_heads, int64_t n_rows,
                                int64_t s_stride_h, int64_t s_stride_r, int64_t block_start,
                                int64_t n_cols, const uint8_t* kv_ok, const int64_t* rows,
                                int64_t k_lo, int64_t k_hi, const uint8_t* extra,
                                int64_t n_extra, int64_t* index, uint8_t* keep,
                                int64_t o_stride_h, int64_t o_stride_r, int64_t col0,
                                void* stream) {
  VEDA_REQUIRE(n_cols >= 1 && n_cols <= kMaxCols, "select_topk: n_cols %lld not in [1, %d]",
               (long long)n_cols, kMaxCols);
  VEDA_REQUIRE(1 <= k_lo && k_lo <= k_hi && k_hi <= n_cols,
               "select_topk: need 1 <= k_lo <= k_hi <= n_cols, got %lld %lld %lld",
               (long long)k_lo, (long long)k_hi, (long long)n_cols);
  VEDA_REQUIRE(block_start >= 0 && n_heads >= 0 && n_rows >= 0, "select_topk: negative size");
  const int64_t items = n_heads * n_rows;
  if (items == 0) return VEDA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const size_t lds = (size_t)kSelWaves * ((n_cols + 63) / 64) * 64 * sizeof(uint64_t);  // <= 64 KB
  static_assert(32 * 64 >= kMaxCols, "select_topk_kernel<32> holds kMaxCols keys per wave");
  const unsigned grid = (unsigned)((items + kSelWaves - 1) / kSelWaves);
  if (n_cols <= 16 * 64)
    select_topk_kernel<16><<<grid, 256, lds, s>>>(
        scores, n_heads, n_rows, s_stride_h, s_stride_r, block_start, (int)n_cols, kv_ok, rows,
        (int)k_lo, (int)k_hi, extra, n_extra, index, keep, o_stride_h, o_stride_r, col0);
  else
    select_topk_kernel<32><<<grid, 256, lds, s>>>(
        scores, n_heads, n_rows, s_stride_h, s_stride_r, block_start, (int)n_cols, kv_ok, rows,
        (int)k_lo, (int)k_hi, extra, n_extra, index, keep, o_stride_h, o_stride_r, col0);
  return check_launch("veda_select_topk");
}

extern "C" int veda_dense_block_mask(const int64_t* index, const uint8_t* keep, int64_t n_heads,
                                     int64_t n_sel, int64_t k_total, const uint8_t* kv_ok,
                                     int64_t n_tiles, int64_t n_video, int global_rows,
                                     uint8_t* mask, void* stream) {
  VEDA_REQUIRE(n_tiles >= 1 && n_tiles <= kMaxTiles, "dense_block_mask: n_tiles %lld > %d",
               (long long)n_tiles, kMaxTiles);
  VEDA_REQUIRE(!global_rows || n_sel == n_video,
               "dense_block_mask: global_rows needs a selection of all video rows");
  const int64_t out_rows = global_rows ? n_tiles : n_sel;
  const int64_t blocks = n_heads * out_rows;
  if (blocks == 0) return VEDA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dense_mask_kernel<<<(unsigned)blocks, 256, 0, s>>>(index, keep, n_sel, k_total, kv_ok,
                                                     (int)n_tiles, n_video, out_rows, mask);
  return check_launch("veda_dense_block_mask");
}

extern "C" int veda_index_lists(const uint8_t* block_mask, int64_t n_heads, int64_t n_rows,
                                int64_t n_tiles, const uint8_t* kv_ok, const uint8_t* full_tile,
                                int32_t* part_cnt, int32_t* part_idx, int32_t* full_cnt,
                                int32_t* full_idx, void* stream) {
  VEDA_REQUIRE(n_tiles >= 1 && n_tiles < (1ll << 31), "index_lists: bad n_tiles");
  const int64_t items = n_heads * n_rows;
  if (items == 0) return VEDA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // widest load every row start and both column tables allow
  auto aligned = [&](int64_t a) {
    return n_tiles % a == 0 && reinterpret_cast<uintptr_t>(block_mask) % a == 0 &&
           reinterpret_cast<uintptr_t>(kv_ok) % a == 0 &&
           reinterpret_cast<uintptr_t>(full_tile) % a == 0;
  };
  const int vec = aligned(16) ? 16 : aligned(4) ? 4 : 1;
  index_lists_kernel<<<(unsigned)((items + kListWaves - 1) / kListWaves), 64 * kListWaves, 0,
                       s>>>(block_mask, items, (int)n_tiles, vec, kv_ok, full_tile, part_cnt,
                            part_idx, full_cnt, full_idx);
  return check_launch("veda_index_lists");
}
