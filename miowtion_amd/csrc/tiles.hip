// Tile permutation kernels: gather (+ pooling, + second moments), scatter
// and the LSE gather. All three are HBM-bound copies.
//
// Work split: one 256-thread workgroup per (tile, group of heads). A wave
// owns 32 of the tile's 128 slots; inside the wave, lane = (head, 16-byte
// chunk of head_dim), so every load and store of a slot's row moves
// `heads_per_group * head_dim * 2` contiguous bytes (heads are adjacent in
// the [S, H, D] input and in the [N, H', D] output). The grid is 1-D with
// the head group fastest: the workgroups that split one tile's rows by head
// run side by side, so each source and destination row is read and written
// whole within a short window (3-6 % faster than tile-fastest order on
// MI355X at 57,720 rows x 48 heads). Pooling statistics are
// reduced in registers over the wave's 32 slots and across the 4 waves
// through LDS, so the tile is read from HBM exactly once (the centred
// variance, when asked for, re-reads it from L2).

#include "veda_common.h"

#include <cstring>
#include <string>

namespace veda {

namespace {
thread_local std::string g_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return VEDA_ELAUNCH;
  }
  return VEDA_OK;
}

namespace {

constexpr int kWaves = 4;
constexpr int kSlotsPerWave = kTile / kWaves;  // 32
constexpr int kCopyWaves = 16;                 // waves of the plain gather and the scatter
constexpr int kPoolUnroll = 4;                 // rows in flight per wave of the pooled gather
constexpr int kPoolOccupancy = 8;              // its waves per SIMD (caps its registers)

struct Row8 {
  uint32_t w[4];  // 8 bf16 values
};

__device__ __forceinline__ Row8 load_row8(const uint16_t* p) {
  u32x4 v = *reinterpret_cast<const u32x4*>(p);
  return Row8{{v[0], v[1], v[2], v[3]}};
}

__device__ __forceinline__ void store_row8(uint16_t* p, const Row8& r) {
  u32x4 v = {r.w[0], r.w[1], r.w[2], r.w[3]};
  *reinterpret_cast<u32x4*>(p) = v;
}


// Streaming forms for rows touched once: the non-temporal hint keeps the
// copy streams from displacing other lines in the caches.
__device__ __forceinline__ Row8 load_row8_nt(const uint16_t* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return Row8{{v[0], v[1], v[2], v[3]}};
}

__device__ __forceinline__ void store_row8_nt(uint16_t* p, const Row8& r) {
  u32x4 v = {r.w[0], r.w[1], r.w[2], r.w[3]};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

__device__ __forceinline__ float elem(const Row8& r, int e) {
  uint32_t w = r.w[e >> 1];
  return bf16_to_f32((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// Gather. Workgroup = (tile, group of heads) with WAVES waves, each on
// 128 / WAVES consecutive slots; lane = (head, 16-byte chunk). More waves
// per tile put more rows in flight per workgroup: the plain copy runs with
// kCopyWaves; the variance pass (pooling with second moments, whose per-wave
// partials go through LDS, [stat][wave][lane][8]) with kWaves.
template <int D, bool POOL, bool SECOND, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) gather_kernel(
    const uint16_t* __restrict__ x, int64_t x_rows, int64_t x_heads,
    int64_t xs, int64_t xh, const int64_t* __restrict__ gather_index,
    const int32_t* __restrict__ slot_valid,
    const int32_t* __restrict__ valid_count, int64_t n_tiles,
    const int64_t* __restrict__ heads, int64_t n_heads,
    uint16_t* __restrict__ out, int64_t os, int64_t oh,
    float* __restrict__ feats, float* __restrict__ sq, float* __restrict__ var) {
  constexpr int kChunks = D / 8;          // 16-byte chunks per head row
  constexpr int kHeadsPerGroup = 64 / kChunks;
  const int n_groups = (int)((n_heads + kHeadsPerGroup - 1) / kHeadsPerGroup);
  const int tile = (int)(blockIdx.x / n_groups);
  const int group = (int)(blockIdx.x % n_groups);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int hl = lane / kChunks;
  const int chunk = lane % kChunks;
  const int64_t hp = (int64_t)group * kHeadsPerGroup + hl;  // h'
  const bool head_ok = hp < n_heads;
  const int64_t head = head_ok ? heads[hp] : 0;
  const bool src_head_ok = head_ok && head >= 0 && head < x_heads;
  constexpr int kSlots = kTile / WAVES;  // slots per wave
  static_assert(!SECOND || WAVES == kWaves, "the variance pass runs on kWaves waves");
  const int64_t slot0 = (int64_t)tile * kTile + wave * kSlots;
  const int count = POOL ? valid_count[tile] : 0;

  float s_sum[8], s_max[8], s_min[8], s_sq[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s_sum[e] = 0.f;
    s_max[e] = -INFINITY;
    s_min[e] = INFINITY;
    s_sq[e] = 0.f;
  }

#pragma unroll 8
  for (int i = 0; i < kSlots; ++i) {
    const int64_t slot = slot0 + i;
    const int64_t src = gather_index[slot];
    const bool ok = slot_valid[slot] != 0 && src_head_ok && src >= 0 && src < x_rows;
    Row8 r = {{0u, 0u, 0u, 0u}};
    // the variance pass re-reads the tile, so it keeps the plain load
    if (ok) r = SECOND ? load_row8(x + src * xs + head * xh + chunk * 8)
                       : load_row8_nt(x + src * xs + head * xh + chunk * 8);
    if (head_ok && out != nullptr) store_row8_nt(out + slot * os + hp * oh + chunk * 8, r);
    if (POOL) {
      const bool real = (wave * kSlots + i) < count;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = elem(r, e);
        s_sum[e] += f;
        if (real) {  // NaN-propagating, as torch's amax / amin
          s_max[e] = __builtin_elementwise_maximum(s_max[e], f);
          s_min[e] = __builtin_elementwise_minimum(s_min[e], f);
        }
        if (SECOND) s_sq[e] += f * f;
      }
    }
  }
  if (!POOL) return;

  // Cross-wave reduction through LDS: [stat][wave][lane][8].
  constexpr int kStats = SECOND ? 4 : 3;
  __shared__ float red[kStats][WAVES][64][8];
  __shared__ float mean_lds[64][8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][wave][lane][e] = s_sum[e];
    red[1][wave][lane][e] = s_max[e];
    red[2][wave][lane][e] = s_min[e];
    if (SECOND) red[kStats - 1][wave][lane][e] = s_sq[e];
  }
  __syncthreads();
  const bool empty = count == 0;
  const float denom = (float)(count > 1 ? count : 1);
  const int64_t fbase = (hp * n_tiles + tile);
  if (wave == 0) {
    float mean[8], mx[8], mn[8], sqv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = red[0][0][lane][e], b = red[1][0][lane][e], c = red[2][0][lane][e];
      float d = SECOND ? red[kStats - 1][0][lane][e] : 0.f;
#pragma unroll
      for (int w = 1; w < WAVES; ++w) {
        a += red[0][w][lane][e];
        b = __builtin_elementwise_maximum(b, red[1][w][lane][e]);
        c = __builtin_elementwise_minimum(c, red[2][w][lane][e]);
        if (SECOND) d += red[kStats - 1][w][lane][e];
      }
      mean[e] = a / denom;
      mean_lds[lane][e] = mean[e];
      mx[e] = empty ? 0.f : b;
      mn[e] = empty ? 0.f : c;
      sqv[e] = empty ? 0.f : d / denom;
      if (empty) mean[e] = 0.f;
    }
    if (head_ok) {
      float* f = feats + fbase * (3 * D) + chunk * 8;
#pragma unroll
      for (int e = 0; e < 8; e += 4) {
        *reinterpret_cast<f32x4*>(f + e) = f32x4{mean[e], mean[e + 1], mean[e + 2], mean[e + 3]};
        *reinterpret_cast<f32x4*>(f + D + e) = f32x4{mx[e], mx[e + 1], mx[e + 2], mx[e + 3]};
        *reinterpret_cast<f32x4*>(f + 2 * D + e) = f32x4{mn[e], mn[e + 1], mn[e + 2], mn[e + 3]};
        if (SECOND)
          *reinterpret_cast<f32x4*>(sq + fbase * D + chunk * 8 + e) =
              f32x4{sqv[e], sqv[e + 1], sqv[e + 2], sqv[e + 3]};
      }
    }
  }
  if (!SECOND) return;
  __syncthreads();
  // Second pass for the centred variance (predictor.py:133-168 computes it
  // two-pass on purpose): sum over real rows of (x - mean)^2.
  float mean[8], acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    mean[e] = mean_lds[lane][e];
    acc[e] = 0.f;
  }
#pragma unroll 8
  for (int i = 0; i < kSlots; ++i) {
    const int64_t slot = slot0 + i;
    if (wave * kSlots + i >= count) break;
    const int64_t src = gather_index[slot];
    const bool ok = slot_valid[slot] != 0 && src_head_ok && src >= 0 && src < x_rows;
    Row8 r = {{0u, 0u, 0u, 0u}};
    if (ok) r = load_row8(x + src * xs + head * xh + chunk * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c = elem(r, e) - mean[e];
      acc[e] += c * c;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[0][wave][lane][e] = acc[e];
  __syncthreads();
  if (wave == 0 && head_ok) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = red[0][0][lane][e];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) a += red[0][w][lane][e];
      v[e] = empty ? 0.f : a / denom;
    }
    float* o = var + fbase * D + chunk * 8;
    *reinterpret_cast<f32x4*>(o) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(o + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// bf16 pairs as int16 pairs whose signed order is the numeric order (the
// magnitude bits of negative values flipped; -0 orders below +0): max and
// min of raw rows in packed integer instructions. The map is an involution.
using s16x2 = short __attribute__((ext_vector_type(2)));

__device__ __forceinline__ s16x2 order_key(s16x2 v) {
  return v ^ ((v >> (short)15) & (short)0x7fff);
}

__device__ __forceinline__ void pool_keys(const Row8& r, s16x2* k_max, s16x2* k_min) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const s16x2 k = order_key(__builtin_bit_cast(s16x2, r.w[w]));
    k_max[w] = __builtin_elementwise_max(k_max[w], k);
    k_min[w] = __builtin_elementwise_min(k_min[w], k);
  }
}

// Gather with first-order pooling: one wave per (tile, group of heads),
// over all 128 slots of the tile, so the pooled statistics stay in the
// lane's registers (no cross-wave reduction, no barrier); the workgroup's
// waves take consecutive head groups of one tile (adjacent bytes of each
// source row).
template <int D>
__global__ void __launch_bounds__(64 * kWaves, kPoolOccupancy) pool_gather_kernel(
    const uint16_t* __restrict__ x, int64_t x_rows, int64_t x_heads,
    int64_t xs, int64_t xh, const int64_t* __restrict__ gather_index,
    const int32_t* __restrict__ slot_valid,
    const int32_t* __restrict__ valid_count, int64_t n_tiles,
    const int64_t* __restrict__ heads, int64_t n_heads,
    uint16_t* __restrict__ out, int64_t os, int64_t oh, float* __restrict__ feats) {
  constexpr int kChunks = D / 8;
  constexpr int kHeadsPerGroup = 64 / kChunks;
  const int n_groups = (int)((n_heads + kHeadsPerGroup - 1) / kHeadsPerGroup);
  const int64_t item =
      (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item >= n_tiles * n_groups) return;
  const int64_t tile = item / n_groups;
  const int group = (int)(item % n_groups);
  const int lane = threadIdx.x & 63;
  const int chunk = lane % kChunks;
  const int64_t hp = (int64_t)group * kHeadsPerGroup + lane / kChunks;
  const bool head_ok = hp < n_heads;
  const int64_t head = head_ok ? heads[hp] : 0;
  const bool src_head_ok = head_ok && head >= 0 && head < x_heads;
  // lanes of a missing head read head 0 of the row and keep zeros
  const int64_t lane_off = (src_head_ok ? head : 0) * xh + chunk * 8;
  const int count = valid_count[tile];
  float s_sum[8];
  s16x2 k_max[4], k_min[4];  // order keys of the bf16 pairs
#pragma unroll
  for (int e = 0; e < 8; ++e) s_sum[e] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    k_max[w] = s16x2{-32768, -32768};
    k_min[w] = s16x2{32767, 32767};
  }
  // 8 slots at a time; the slots before `count` are the tile's real rows
  // (every layout puts them first): max / min over those, the sum over all
  // (the padding rows are zero).
#pragma unroll 1
  for (int i0 = 0; i0 < kTile; i0 += kPoolUnroll) {
    // wave-uniform slots: the index reads are scalar loads, all issued first
    int64_t src[kPoolUnroll];
    bool ok[kPoolUnroll];
#pragma unroll
    for (int j = 0; j < kPoolUnroll; ++j) {
      const int64_t slot = tile * kTile + i0 + j;
      src[j] = gather_index[slot];
      ok[j] = slot_valid[slot] != 0;
    }
    Row8 r[kPoolUnroll];
#pragma unroll
    for (int j = 0; j < kPoolUnroll; ++j) {
      r[j] = Row8{{0u, 0u, 0u, 0u}};
      if (ok[j] && src[j] >= 0 && src[j] < x_rows)
        r[j] = load_row8_nt(x + src[j] * xs + lane_off);
    }
    if (!src_head_ok) {
#pragma unroll
      for (int j = 0; j < kPoolUnroll; ++j) r[j] = Row8{{0u, 0u, 0u, 0u}};
    }
#pragma unroll
    for (int j = 0; j < kPoolUnroll; ++j)
      if (head_ok && out != nullptr)
        store_row8_nt(out + (tile * kTile + i0 + j) * os + hp * oh + chunk * 8, r[j]);
#pragma unroll
    for (int j = 0; j < kPoolUnroll; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_sum[e] += elem(r[j], e);
      if (i0 + j < count) pool_keys(r[j], k_max, k_min);  // wave-uniform branch
    }
  }
  if (!head_ok) return;
  const bool empty = count == 0;
  const float denom = (float)(count > 1 ? count : 1);
  float* f = feats + (hp * n_tiles + tile) * (3 * D) + chunk * 8;
  float s_max[8], s_min[8];
  {
    Row8 mx, mn;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mx.w[w] = __builtin_bit_cast(uint32_t, order_key(k_max[w]));  // the key map is its own inverse
      mn.w[w] = __builtin_bit_cast(uint32_t, order_key(k_min[w]));
    }
    // A NaN of either sign among the real rows makes both max and min NaN,
    // as torch's amax / amin propagate it: a +NaN key orders above +inf's
    // and a -NaN key below -inf's, so one of the two accumulators holds it.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = elem(mx, e), b = elem(mn, e);
      const bool nan = a != a || b != b;
      s_sum[e] = empty ? 0.f : s_sum[e] / denom;
      s_max[e] = empty ? 0.f : nan ? __builtin_nanf("") : a;
      s_min[e] = empty ? 0.f : nan ? __builtin_nanf("") : b;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e += 4) {
    *reinterpret_cast<f32x4*>(f + e) = f32x4{s_sum[e], s_sum[e + 1], s_sum[e + 2], s_sum[e + 3]};
    *reinterpret_cast<f32x4*>(f + D + e) = f32x4{s_max[e], s_max[e + 1], s_max[e + 2], s_max[e + 3]};
    *reinterpret_cast<f32x4*>(f + 2 * D + e) =
        f32x4{s_min[e], s_min[e + 1], s_min[e + 2], s_min[e + 3]};
  }
}

template <int D, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) scatter_kernel(
    const uint16_t* __restrict__ tiled, int64_t ts, int64_t th,
    const int64_t* __restrict__ scatter_index,
    const int32_t* __restrict__ slot_valid, const int64_t* __restrict__ heads,
    int64_t n_heads, uint16_t* __restrict__ out, int64_t out_rows,
    int64_t out_heads, int64_t os, int64_t oh) {
  constexpr int kChunks = D / 8;
  constexpr int kHeadsPerGroup = 64 / kChunks;
  const int n_groups = (int)((n_heads + kHeadsPerGroup - 1) / kHeadsPerGroup);
  const int tile = (int)(blockIdx.x / n_groups);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t hp = (int64_t)(blockIdx.x % n_groups) * kHeadsPerGroup + lane / kChunks;
  const int chunk = lane % kChunks;
  if (hp >= n_heads) return;
  const int64_t head = heads[hp];
  if (head < 0 || head >= out_heads) return;
  constexpr int kSlots = kTile / WAVES;
  const int64_t slot0 = (int64_t)tile * kTile + wave * kSlots;
#pragma unroll 8
  for (int i = 0; i < kSlots; ++i) {
    const int64_t slot = slot0 + i;
    const int64_t dst = scatter_index[slot];
    if (slot_valid[slot] == 0 || dst < 0 || dst >= out_rows) continue;
    Row8 r = load_row8_nt(tiled + slot * ts + hp * th + chunk * 8);
    store_row8_nt(out + dst * os + head * oh + chunk * 8, r);
  }
}

__global__ void gather_lse_kernel(const float* __restrict__ lse, int64_t rows,
                                  int64_t n_src_heads, int64_t ls, int64_t lh,
                                  const int64_t* __restrict__ gather_index,
                                  const int32_t* __restrict__ slot_valid,
                                  int64_t n_slots, const int64_t* __restrict__ heads,
                                  int64_t n_heads, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_slots * n_heads) return;
  const int64_t s = i / n_heads, hp = i % n_heads;
  const int64_t src = gather_index[s];
  const int64_t head = heads[hp];
  float v = 0.f;
  if (slot_valid[s] != 0 && src >= 0 && src < rows && head >= 0 && head < n_src_heads)
    v = lse[src * ls + head * lh];
  out[i] = v;
}

// Tile summaries for the zero-order compensation: per (key tile, head) the
// mean of K over the tile's real rows (divided by max(count, 1)) and the
// sum of V over them, both rounded to bf16 (the summaries of
// miowtion/kernels/compensation_triton.py:80-99; real rows are the first
// valid_count[t] slots). Workgroup = (tile, 4 heads): lane (head, 16-byte
// chunk), wave = 32 slots; fp32 sums, reduced across waves through LDS.
__global__ void __launch_bounds__(256) summary_kernel(
    const uint16_t* __restrict__ k, int64_t ks, int64_t kh, const uint16_t* __restrict__ v,
    int64_t vs, int64_t vh, const int32_t* __restrict__ valid_count, int64_t n_heads,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t cs, int64_t ch) {
  constexpr int kChunks = 16;  // D = 128
  const int tile = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t head = (int64_t)blockIdx.y * 4 + lane / kChunks;
  const int chunk = lane % kChunks;
  const bool head_ok = head < n_heads;
  const int count = min(max(valid_count[tile], 0), kTile);
  float sk[8], sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sk[e] = sv[e] = 0.f;
  const int first = wave * kSlotsPerWave, last = min(first + kSlotsPerWave, count);
  for (int i = first; i < last && head_ok; ++i) {
    const int64_t row = (int64_t)tile * kTile + i;
    const Row8 a = load_row8(k + row * ks + head * kh + chunk * 8);
    const Row8 b = load_row8(v + row * vs + head * vh + chunk * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sk[e] += elem(a, e);
      sv[e] += elem(b, e);
    }
  }
  __shared__ float red[2][kWaves][64][8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][wave][lane][e] = sk[e];
    red[1][wave][lane][e] = sv[e];
  }
  __syncthreads();
  if (wave != 0 || !head_ok) return;
  const float denom = (float)(count > 1 ? count : 1);
  Row8 ok = {{0u, 0u, 0u, 0u}}, ov = {{0u, 0u, 0u, 0u}};
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      a0 += red[0][w][lane][e];
      a1 += red[0][w][lane][e + 1];
      b0 += red[1][w][lane][e];
      b1 += red[1][w][lane][e + 1];
    }
    ok.w[e >> 1] = pack_bf16x2(a0 / denom, a1 / denom);
    ov.w[e >> 1] = pack_bf16x2(b0, b1);
  }
  store_row8(kc + (int64_t)tile * cs + head * ch + chunk * 8, ok);
  store_row8(vc + (int64_t)tile * cs + head * ch + chunk * 8, ov);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" const char* veda_last_error(void) { return g_error.c_str(); }

extern "C" int veda_abi_version(void) { return 5; }

extern "C" int veda_gather_tiles(const void* x, int64_t x_rows, int64_t x_heads,
                                 int64_t x_stride_s, int64_t x_stride_h,
                                 const int64_t* gather_index, const int32_t* slot_valid,
                                 const int32_t* valid_count, int64_t n_tiles,
                                 const int64_t* heads, int64_t n_heads, int64_t head_dim,
                                 void* out, int64_t out_stride_s, int64_t out_stride_h,
                                 float* feats, float* sq, float* var, void* stream) {
  VEDA_REQUIRE(head_dim == 64 || head_dim == 128, "gather: head_dim must be 64 or 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(n_tiles >= 0 && n_heads >= 0, "gather: negative size");
  VEDA_REQUIRE(x_stride_s % 8 == 0 && x_stride_h % 8 == 0 && out_stride_s % 8 == 0 &&
                   out_stride_h % 8 == 0 && aligned16(x) && aligned16(out),
               "gather: rows must be 16-byte aligned (strides multiple of 8 elements)");
  VEDA_REQUIRE((sq == nullptr) == (var == nullptr), "gather: sq and var go together");
  VEDA_REQUIRE(feats != nullptr || sq == nullptr, "gather: second moments need pooling");
  VEDA_REQUIRE(feats == nullptr || valid_count != nullptr, "gather: pooling needs valid_count");
  if (n_tiles == 0 || n_heads == 0) return VEDA_OK;
  const int hpg = head_dim == 128 ? 4 : 8;
  const int64_t n_wg = n_tiles * ((n_heads + hpg - 1) / hpg);
  VEDA_REQUIRE(n_wg <= INT32_MAX, "gather: %lld tiles x head groups exceed one launch",
               (long long)n_wg);
  dim3 grid((unsigned)n_wg);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto xx = static_cast<const uint16_t*>(x);
  auto oo = static_cast<uint16_t*>(out);
#define VEDA_GATHER(D, P, S2, W)                                                              \
  gather_kernel<D, P, S2, W><<<grid, 64 * W, 0, s>>>(                                          \
      xx, x_rows, x_heads, x_stride_s, x_stride_h, gather_index, slot_valid, valid_count,      \
      n_tiles, heads, n_heads, oo, out_stride_s, out_stride_h, feats, sq, var)
#define VEDA_POOL_GATHER(D)                                                                   \
  pool_gather_kernel<D><<<(unsigned)((n_wg + kWaves - 1) / kWaves), 64 * kWaves, 0, s>>>(      \
      xx, x_rows, x_heads, x_stride_s, x_stride_h, gather_index, slot_valid, valid_count,      \
      n_tiles, heads, n_heads, oo, out_stride_s, out_stride_h, feats)
  if (head_dim == 128) {
    if (!feats) VEDA_GATHER(128, false, false, kCopyWaves);
    else if (!sq) VEDA_POOL_GATHER(128);
    else VEDA_GATHER(128, true, true, kWaves);
  } else {
    if (!feats) VEDA_GATHER(64, false, false, kCopyWaves);
    else if (!sq) VEDA_POOL_GATHER(64);
    else VEDA_GATHER(64, true, true, kWaves);
  }
#undef VEDA_GATHER
#undef VEDA_POOL_GATHER
  return check_launch("veda_gather_tiles");
}

extern "C" int veda_scatter_tiles(const void* tiled, int64_t tiled_stride_s,
                                  int64_t tiled_stride_h, const int64_t* scatter_index,
                                  const int32_t* slot_valid, int64_t n_tiles,
                                  const int64_t* heads, int64_t n_heads, int64_t head_dim,
                                  void* out, int64_t out_rows, int64_t out_heads,
                                  int64_t out_stride_s, int64_t out_stride_h, void* stream) {
  VEDA_REQUIRE(head_dim == 64 || head_dim == 128, "scatter: head_dim must be 64 or 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(tiled_stride_s % 8 == 0 && tiled_stride_h % 8 == 0 && out_stride_s % 8 == 0 &&
                   out_stride_h % 8 == 0 && aligned16(tiled) && aligned16(out),
               "scatter: rows must be 16-byte aligned (strides multiple of 8 elements)");
  if (n_tiles == 0 || n_heads == 0) return VEDA_OK;
  const int hpg = head_dim == 128 ? 4 : 8;
  const int64_t n_wg = n_tiles * ((n_heads + hpg - 1) / hpg);
  VEDA_REQUIRE(n_wg <= INT32_MAX, "scatter: %lld tiles x head groups exceed one launch",
               (long long)n_wg);
  dim3 grid((unsigned)n_wg);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto tt = static_cast<const uint16_t*>(tiled);
  auto oo = static_cast<uint16_t*>(out);
  if (head_dim == 128)
    scatter_kernel<128, kCopyWaves><<<grid, 64 * kCopyWaves, 0, s>>>(
        tt, tiled_stride_s, tiled_stride_h, scatter_index, slot_valid, heads, n_heads, oo,
        out_rows, out_heads, out_stride_s, out_stride_h);
  else
    scatter_kernel<64, kCopyWaves><<<grid, 64 * kCopyWaves, 0, s>>>(
        tt, tiled_stride_s, tiled_stride_h, scatter_index, slot_valid, heads, n_heads, oo,
        out_rows, out_heads, out_stride_s, out_stride_h);
  return check_launch("veda_scatter_tiles");
}

extern "C" int veda_gather_lse(const float* lse, int64_t lse_rows, int64_t lse_heads,
                               int64_t lse_stride_s, int64_t lse_stride_h,
                               const int64_t* gather_index, const int32_t* slot_valid,
                               int64_t n_slots, const int64_t* heads, int64_t n_heads,
                               float* out, void* stream) {
  VEDA_REQUIRE(n_slots >= 0 && n_heads >= 0, "gather_lse: negative size");
  const int64_t total = n_slots * n_heads;
  if (total == 0) return VEDA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  gather_lse_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
      lse, lse_rows, lse_heads, lse_stride_s, lse_stride_h, gather_index, slot_valid, n_slots,
      heads, n_heads, out);
  return check_launch("veda_gather_lse");
}

extern "C" int veda_tile_summaries(const void* k, int64_t k_stride_s, int64_t k_stride_h,
                                   const void* v, int64_t v_stride_s, int64_t v_stride_h,
                                   const int32_t* valid_count, int64_t n_tiles, int64_t n_heads,
                                   int64_t head_dim, void* kc, void* vc, int64_t c_stride_s,
                                   int64_t c_stride_h, void* stream) {
  VEDA_REQUIRE(head_dim == 128, "tile_summaries: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(n_tiles >= 0 && n_heads >= 0, "tile_summaries: negative size");
  VEDA_REQUIRE(aligned16(k) && aligned16(v) && aligned16(kc) && aligned16(vc) &&
                   k_stride_s % 8 == 0 && k_stride_h % 8 == 0 && v_stride_s % 8 == 0 &&
                   v_stride_h % 8 == 0 && c_stride_s % 8 == 0 && c_stride_h % 8 == 0,
               "tile_summaries: rows must be 16-byte aligned");
  if (n_tiles == 0 || n_heads == 0) return VEDA_OK;
  dim3 grid((unsigned)n_tiles, (unsigned)((n_heads + 3) / 4));
  summary_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(k), k_stride_s, k_stride_h, static_cast<const uint16_t*>(v),
      v_stride_s, v_stride_h, valid_count, n_heads, static_cast<uint16_t*>(kc),
      static_cast<uint16_t*>(vc), c_stride_s, c_stride_h);
  return check_launch("veda_tile_summaries");
}
