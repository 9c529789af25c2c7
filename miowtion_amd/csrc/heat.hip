// Teacher block heat for gfx950: per (head, query tile, key tile) the block's
// softmax mass ('sum') or peak probability ('max') from the dense LSE.
//
// Workgroup = (head, query tile, run of 16 key tiles), 4 waves; wave w owns
// query rows 32w .. 32w+31 of the tile and keeps them in registers as the
// B operand of S^T = K Q^T (v_mfma_f32_32x32x16_bf16), so each lane holds one
// query row and 64 of the 128 keys of a block. K tiles are double-buffered
// in LDS (16-byte XOR swizzle, as in the attention kernel) together with a
// 128-bit key-validity mask; the next tile is loaded while the current one
// is reduced. Only one fp32 value per block leaves the workgroup.

#include "veda_common.h"

namespace veda {
namespace {

constexpr int kD = 128;
constexpr int kHeatThreads = 256;
constexpr int kTilesPerGroup = 16;
constexpr int kKBytes = kTile * kD * 2;  // 32 KB
constexpr float kLog2e = 1.4426950408889634f;

struct HeatParams {
  const uint16_t* q;
  const uint16_t* k;
  int64_t qs, qh, ks, kh;
  const float* lse;
  int64_t ls, lh;
  const int32_t* slot_valid;
  const int64_t* q_tiles;
  int64_t n_q, n_tiles, n_heads, n_groups;
  int reduce;  // 0 sum, 1 max
  float scale;
  float* heat;
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ void load_k(const HeatParams& p, int64_t head, int64_t j, int tid,
                                       u32x4 (&st)[8], int& valid) {
  const int64_t row0 = j * kTile;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = tid + 256 * u;
    const int row = c >> 4, ch = c & 15;
    st[u] = *reinterpret_cast<const u32x4*>(p.k + (row0 + row) * p.ks + head * p.kh + ch * 8);
  }
  valid = tid < kTile ? p.slot_valid[row0 + tid] : 0;
}

__device__ __forceinline__ void store_k(uint8_t* buf, uint64_t* vmask, int tid,
                                        const u32x4 (&st)[8], int valid) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = tid + 256 * u;
    const int row = c >> 4, ch = c & 15;
    *reinterpret_cast<u32x4*>(buf + row * 256 + ((ch ^ (row & 15)) << 4)) = st[u];
  }
  const uint64_t b = __ballot(valid != 0);
  if (tid < kTile && (tid & 63) == 0) vmask[tid >> 6] = b;
}

__global__ void __launch_bounds__(kHeatThreads) heat_kernel(HeatParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t kbuf[2][kKBytes];
  __shared__ uint64_t vmask[2][2];
  __shared__ float part[4][kTilesPerGroup];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 31, hi = lane >> 5;
  const int64_t item = blockIdx.x;
  const int64_t g = item % p.n_groups;
  const int64_t hr = item / p.n_groups;
  const int64_t r = hr % p.n_q;
  const int64_t head = hr / p.n_q;
  const int64_t qt = p.q_tiles[r];
  const int64_t j0 = g * kTilesPerGroup;
  const int64_t j1 = j0 + kTilesPerGroup < p.n_tiles ? j0 + kTilesPerGroup : p.n_tiles;
  const int nt = (int)(j1 - j0);
  if (qt < 0 || qt >= p.n_tiles) {  // not a query tile of this layout: no heat
    if (tid < nt) p.heat[(head * p.n_q + r) * p.n_tiles + j0 + tid] = 0.f;
    return;
  }
  const int64_t qrow = qt * kTile + 32 * wave + li;

  bf16x8 qf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    qf[s] = as_bf16x8(*reinterpret_cast<const u32x4*>(p.q + qrow * p.qs + head * p.qh + 16 * s + 8 * hi));
  const bool row_ok = p.slot_valid[qrow] != 0;
  const float lse = p.lse[qrow * p.ls + head * p.lh];
  const float lse2 = row_ok ? lse * kLog2e : INFINITY;   // sum: exp2 domain
  const float lse_n = row_ok ? lse : INFINITY;           // max: natural domain
  const float c2 = p.scale * kLog2e;

  u32x4 st[8];
  int valid;
  load_k(p, head, j0, tid, st, valid);
  store_k(kbuf[0], vmask[0], tid, st, valid);
  __syncthreads();
  for (int t = 0; t < nt; ++t) {
    if (t + 1 < nt) load_k(p, head, j0 + t + 1, tid, st, valid);
    const uint8_t* kb = kbuf[t & 1];
    const uint64_t vm[2] = {vmask[t & 1][0], vmask[t & 1][1]};
    float acc = p.reduce ? -INFINITY : 0.f;
#pragma unroll
    for (int t2 = 0; t2 < 4; ++t2) {
      f32x16 sacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
      const int krow = 32 * t2 + li;
      const uint8_t* kr = kb + krow * 256;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int ch = 2 * s + hi;
        bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4*>(kr + ((ch ^ (krow & 15)) << 4)));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], sacc, 0, 0, 0);
      }
      // Register e holds key 32 t2 + 8 (e / 4) + 4 hi + e % 4.
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = 32 * t2 + 8 * (e >> 2) + 4 * hi + (e & 3);
        const bool kv = (vm[key >> 6] >> (key & 63)) & 1ull;
        if (p.reduce) {
          acc = kv ? fmaxf(acc, sacc[e]) : acc;
        } else {
          acc += kv ? __builtin_amdgcn_exp2f(sacc[e] * c2 - lse2) : 0.f;
        }
      }
    }
    float v;
    if (p.reduce) {
      // Row max over the block, rounded to bf16 like the reference's bf16
      // scores (rounding is monotonic, so rounding the max is rounding all).
      float rm = fmaxf(acc, __shfl_xor(acc, 32, 64));
      if (rm != -INFINITY) rm = bf16_to_f32(f32_to_bf16(rm));
      v = rm * p.scale - lse_n;
      if (rm == -INFINITY || !row_ok) v = -INFINITY;
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    } else {
      v = acc;
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    }
    if (lane == 0) part[wave][t] = v;
    if (t + 1 < nt) store_k(kbuf[(t + 1) & 1], vmask[(t + 1) & 1], tid, st, valid);
    __syncthreads();
  }
  if (tid < nt) {
    float v = part[0][tid];
    if (p.reduce) {
      for (int w = 1; w < 4; ++w) v = fmaxf(v, part[w][tid]);
      v = v == -INFINITY ? 0.f : expf(v);
    } else {
      for (int w = 1; w < 4; ++w) v += part[w][tid];
    }
    p.heat[(head * p.n_q + r) * p.n_tiles + j0 + tid] = v;
  }
}

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" int veda_block_heat(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                               const void* k, int64_t k_stride_s, int64_t k_stride_h,
                               const float* lse, int64_t lse_stride_s, int64_t lse_stride_h,
                               const int32_t* slot_valid, const int64_t* q_tiles, int64_t n_q,
                               int64_t n_tiles, int64_t n_heads, int64_t head_dim, int reduce,
                               float scale, float* heat, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_heat: head_dim must be 128, got %lld", (long long)head_dim);
  VEDA_REQUIRE(reduce == 0 || reduce == 1, "block_heat: reduce must be 0 (sum) or 1 (max)");
  VEDA_REQUIRE(q_stride_s % 8 == 0 && q_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   k_stride_h % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(k) & 15) == 0,
               "block_heat: rows must be 16-byte aligned");
  VEDA_REQUIRE(n_q >= 0 && n_tiles >= 0 && n_heads >= 0, "block_heat: negative size");
  if (n_q == 0 || n_tiles == 0 || n_heads == 0) return VEDA_OK;
  HeatParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.qs = q_stride_s; p.qh = q_stride_h; p.ks = k_stride_s; p.kh = k_stride_h;
  p.lse = lse; p.ls = lse_stride_s; p.lh = lse_stride_h;
  p.slot_valid = slot_valid; p.q_tiles = q_tiles;
  p.n_q = n_q; p.n_tiles = n_tiles; p.n_heads = n_heads;
  p.n_groups = (n_tiles + kTilesPerGroup - 1) / kTilesPerGroup;
  p.reduce = reduce; p.scale = scale; p.heat = heat;
  const int64_t items = n_heads * n_q * p.n_groups;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  heat_kernel<<<(unsigned)items, kHeatThreads, 0, s>>>(p);
  return check_launch("veda_block_heat");
}
