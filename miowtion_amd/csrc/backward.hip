// Block-sparse flash-attention backward for gfx950 (head_dim 128, bf16
// operands and gradients, fp32 accumulation): dQ, dK, dV of
//   O = softmax(Q K^T * scale over the kept key tiles' valid keys) V
// given dO and the forward's per-row log-sum-exp.
//
// Three kernels, none of them atomic: every gradient row is written by
// exactly one workgroup, so the result does not depend on scheduling.
//   bwd_stats_kernel  per 64-row step of every query tile: the LSE in log2
//                     units (+inf for a row with no key, so its P is 0) and
//                     D = rowsum(dO * O) - dLSE in fp32 (the LSE output's
//                     gradient adds dLSE * P to dS), stored as a 1 KB record
//                     [lse2 x 64 | -D x 64 | 0 x 128] that one wave loads
//                     into LDS with one DMA. -D is the initial accumulator
//                     of the dP products, so they produce dP - D directly.
//   dq_kernel         workgroup = (head, query tile), walking the forward
//                     block lists (the key tiles of the row).
//   dkv_kernel        workgroup = (head, key tile), walking the transposed
//                     lists (the query tiles of the column).
// Per pair of a 64-row and a 64-key half:
//   P  = exp2(S * scale * log2(e) - lse2)   (0 past the key tile's valid count)
//   dP = dO V^T,  dS = P * (dP - D)
//   dQ += dS K * scale,  dK += dS^T Q * scale,  dV += P^T dO
// dq_kernel forms the transposed products (S^T = K Q^T: a lane owns one
// query row, as in the forward kernel), dkv_kernel the plain ones
// (S = Q K^T: a lane owns one key), so that in each kernel P or dS goes from
// the MFMA accumulators straight into the B operand of its own accumulation
// (the MFMA contracts over k in any order, so a lane supplies the rows in the
// order in which its accumulators hold them: 16 s + 4 h + {0..3, 8..11} for
// lane half h of a 32x32 product, 16 (e / 4) + 4 g + e % 4 for lane group g
// of a 16x16 one).
//
// LDS rows are 256 bytes (128 bf16). Logical 16-byte chunk c of row r sits at
// position c ^ swz(r) (K and V in dq_kernel), swz(r) = 4 (r mod 4) +
// (r / 4 mod 4), or c ^ swzk(r) (Q and dO in dkv_kernel, whose read patterns
// differ). Each kernel's read patterns are free of bank conflicts with its
// swizzle (the dkv_kernel comment gives gfx950's lane grouping). Tiles go
// from HBM into LDS with global_load_lds_dwordx4 (the swizzle is applied by
// the choice of source address), double-buffered: step u + 1 loads while
// step u computes.

#include <mutex>

#include <type_traits>

#include "veda_common.h"
#include "veda_pipeline.h"

namespace veda {
namespace {

constexpr int kD = 128;
constexpr int kMaxTiles = 2048;                  // tiles per list row (FA4's cap)
constexpr int kRecFloats = 256;                  // stats record: 64 lse2, 64 -D, the zero
                                                 // flag, zeros
constexpr int kZeroFlag = 128;                   // 1 if every row has dO = 0 and D = 0
constexpr int kHiZeroFlag = 129;                 // 1 if rows 32 .. 63 have dO = 0 and D = 0
constexpr int kRecBytes = kRecFloats * 4;
constexpr int kDqThreads = 256;
constexpr int kDkvThreads = 512;
constexpr int kSlot = 2 * kHalfBytes;            // K + V (dq) or Q + dO (dkv) of a step
constexpr float kLog2e = 1.4426950408889634f;

typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  int64_t qs, qh, ks, kh, vs, vh, os, oh, dos, doh;
  const float* lse;
  int64_t lse_sh, lse_ss;
  const float* dlse;  // NULL: the LSE output carries no gradient
  int64_t dlse_sh, dlse_ss;
  int64_t n_heads, n_q_tiles, n_k_tiles;
  // forward lists: row = (head, query tile), entries = key tiles
  const int32_t* full_cnt;
  const int32_t* full_idx;
  const int32_t* part_cnt;
  const int32_t* part_idx;
  int64_t list_ld;
  // transposed lists: row = (head, key tile), entries = query tiles
  const int32_t* full_cnt_t;
  const int32_t* full_idx_t;
  const int32_t* part_cnt_t;
  const int32_t* part_idx_t;
  int64_t list_ld_t;
  const int32_t* valid_count;
  float scale, scale_log2;
  float* stats;  // [H'][2 R] records
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t dqs, dqh, dks, dkh, dvs, dvh;
  int64_t front;  // the last `front` query tiles (dQ) and key tiles (dK, dV) go first
};

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ int clamp_vc(int32_t vc) { return min(max(vc, 0), kTile); }

// Byte offset (from the step's first row) that lane `lane` of 1 KB segment
// `seg` loads: row 4 seg + lane / 16, LDS position lane % 16, which holds
// logical chunk (lane % 16) ^ swz(row).
__device__ __forceinline__ uint32_t seg_offset(int seg, int lane, int64_t stride) {
  const int row = 4 * seg + (lane >> 4), pc = lane & 15;
  return (uint32_t)((row * stride + ((pc ^ swz(row)) << 3)) * 2);
}

// Per-lane LDS byte offsets of the fragment reads of a 64-row region.
//   row[s]:  A fragment of rows li (+ 32 g), chunk 2 s + hi (16-byte read).
//   tr[dt][e]: transposed read of rows 4 hi + i / 4 + 8 e (+ 16 kk + 32 g),
//            head-dims 32 dt + 16 dh + 4 (i % 4) .. + 3 (i = lane % 16,
//            dh = lane / 16 % 2): lane (dh, i) receives the 4 rows at
//            head-dim 32 dt + 16 dh + i, i.e. row m = lane % 32 of A^T.
// The +32 g rows, +16 kk rows (4096 B) and region offsets are added as
// immediates: none of them changes swz.
struct Frag {
  uint32_t row[8];
  uint32_t tr[4][2];
};

__device__ __forceinline__ Frag frag_offsets(int lane) {
  Frag f;
  const int li = lane & 31, hi = lane >> 5;
#pragma unroll
  for (int s = 0; s < 8; ++s) f.row[s] = li * 256 + (((2 * s + hi) ^ swz(li)) << 4);
  const int i = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 4 * hi + (i >> 2) + 8 * e;
      const int c = 4 * dt + 2 * dh + ((i >> 1) & 1);
      f.tr[dt][e] = r * 256 + ((c ^ swz(r)) << 4) + 8 * (i & 1);
    }
  return f;
}

__device__ __forceinline__ u32x4 lds16(const lds_u8* p) {
  return *reinterpret_cast<const lds_u32x4*>(p);
}

// A^T fragment (32 head-dims x 16 rows) of rows kk * 16 of the region at `base`.
__device__ __forceinline__ bf16x8 tr_frag(const lds_u8* base, const Frag& f, int dt, int kk) {
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + kk * 4096 + f.tr[dt][0]));
  const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + kk * 4096 + f.tr[dt][1]));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7));
}

// The 16 accumulator values of a lane as the two B-operand k-steps
// (rows 16 kk + 4 hi + {0..3, 8..11}), bf16.
__device__ __forceinline__ void pack_b(const float (&x)[16], u32x4 (&pk)[2]) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int m = 0; m < 4; ++m) pk[kk][m] = pack_bf16x2(x[8 * kk + 2 * m], x[8 * kk + 2 * m + 1]);
}

// Wave 0 of a workgroup: the steps (target << 1 | half) of the full list,
// then of the partial list, in list order; halves(t) = which 64-row halves
// of target t are steps (bit 0: the first, bit 1: the second; 0 drops the
// entry) and which of those are "upper-zero" steps (bit 2: the first, bit 3:
// the second), which go to the back of `steps` (entry k of them at
// 2 kMaxTiles - 1 - k), also in list order. Returns the count of the others;
// n_hz receives the count of the upper-zero steps.
template <class Halves>
__device__ int build_steps(const int32_t* fl, int nf, const int32_t* pl, int np, int lane,
                           uint16_t* steps, Halves halves, int& n_hz) {
  int n = 0, nz = 0;
  const int total = nf + np;
  auto below = [](uint64_t b) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0));
  };
  for (int i0 = 0; i0 < total; i0 += 64) {
    const int i = i0 + lane;
    int t = 0, h = 0;
    if (i < total) {
      t = i < nf ? fl[i] : pl[i - nf];
      h = halves(t);
    }
    const bool f0 = (h & 1) && !(h & 4), f1 = (h & 2) && !(h & 8);  // the others
    const bool z0 = (h & 1) && (h & 4), z1 = (h & 2) && (h & 8);    // upper-zero
    const uint64_t bf0 = __ballot(f0), bf1 = __ballot(f1), bz0 = __ballot(z0), bz1 = __ballot(z1);
    const int rf = n + below(bf0) + below(bf1), rz = nz + below(bz0) + below(bz1);
    if (f0) steps[rf] = (uint16_t)(t << 1);
    if (f1) steps[rf + (int)f0] = (uint16_t)((t << 1) | 1);
    if (z0) steps[2 * kMaxTiles - 1 - rz] = (uint16_t)(t << 1);
    if (z1) steps[2 * kMaxTiles - 1 - (rz + (int)z0)] = (uint16_t)((t << 1) | 1);
    n += __builtin_popcountll(bf0) + __builtin_popcountll(bf1);
    nz += __builtin_popcountll(bz0) + __builtin_popcountll(bz1);
  }
  n_hz = nz;
  return n;
}

// Clamped entry counts of list row `lr` (at most kMaxTiles together).
__device__ __forceinline__ void list_counts(const int32_t* fc, const int32_t* pc, int64_t lr,
                                            int64_t ld, int& nf, int& np) {
  const int cap = (int)min(ld, (int64_t)kMaxTiles);
  nf = min(max(fc[lr], 0), cap);
  np = min(max(pc[lr], 0), min(cap, kMaxTiles - nf));
}

// ---------------------------------------------------------------------------
// Row statistics. Block = one 64-row record; 16 lanes per row, each lane 8
// head-dims.

__global__ void __launch_bounds__(256) bwd_stats_kernel(BwdParams p) {
  const int64_t rec = blockIdx.x;
  const int64_t per_head = 2 * p.n_q_tiles;
  const int64_t head = rec / per_head, st = rec % per_head;
  const int tid = threadIdx.x, sub = tid & 15;
  float* out = p.stats + rec * kRecFloats;
  bool live = false, live_hi = false;  // a non-zero dO element or D among this thread's
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int rr = 16 * it + (tid >> 4);
    const int64_t row = st * 64 + rr;
    const u32x4 a = ld16(p.o + row * p.os + head * p.oh + 8 * sub);
    const u32x4 b = ld16(p.dout + row * p.dos + head * p.doh + 8 * sub);
    const bool nz = ((b[0] | b[1] | b[2] | b[3]) & 0x7FFF7FFFu) != 0;  // +-0 count as zero
    live |= nz;
    if (it >= 2) live_hi |= nz;
    float acc = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      acc = fmaf(bf16_to_f32(a[m] & 0xffffu), bf16_to_f32(b[m] & 0xffffu), acc);
      acc = fmaf(bf16_to_f32(a[m] >> 16), bf16_to_f32(b[m] >> 16), acc);
    }
    acc += __shfl_xor(acc, 8, 16);
    acc += __shfl_xor(acc, 4, 16);
    acc += __shfl_xor(acc, 2, 16);
    acc += __shfl_xor(acc, 1, 16);
    if (sub == 0) {
      const float l = p.lse[head * p.lse_sh + row * p.lse_ss];
      out[rr] = l == -INFINITY ? INFINITY : l * kLog2e;
      const float nd = p.dlse != nullptr ? p.dlse[head * p.dlse_sh + row * p.dlse_ss] - acc : -acc;
      out[64 + rr] = nd;
      live |= nd != 0.f;  // NaN too
      if (it >= 2) live_hi |= nd != 0.f;
    }
  }
  const bool zero = __syncthreads_and(!live) != 0;
  const bool zero_hi = __syncthreads_and(!live_hi) != 0;
  if (tid < 128)
    out[kZeroFlag + tid] = (tid == 0 && zero) || (tid == 1 && zero_hi) ? 1.f : 0.f;
}

// ---------------------------------------------------------------------------
// dQ. Workgroup = (head, query tile), 4 waves, two workgroups per CU (74 KB
// of LDS each; their waves are not tied by a barrier, so the two waves of a
// SIMD fill each other's stalls). Wave w owns query rows 32 w .. + 31 (one
// per lane, as B = Q^T and dO^T fragments in registers) and both 32-key
// halves of every 64-key step. Per half: S^T = K Q^T and dP^T = V dO^T (8
// MFMAs each, A = K / V rows from LDS), dS^T, then dQ^T += K^T dS^T (8
// MFMAs, A = transposed K reads).

__global__ void __launch_bounds__(kDqThreads, 2) dq_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[2][kSlot];
  __shared__ uint16_t steps[2 * kMaxTiles];
  __shared__ uint8_t tvc[kMaxTiles];
  __shared__ int32_t step_total;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 31, hi = lane >> 5;
  int64_t head, r;
  front_first(blockIdx.x, p.n_heads, p.n_q_tiles, p.front, head, r);
  const int64_t qrow = r * kTile + 32 * wave + li;
  const int nk = (int)p.n_k_tiles;

  for (int j = tid; j < nk; j += kDqThreads) tvc[j] = (uint8_t)clamp_vc(p.valid_count[j]);
  if (wave == 0) {
    const int64_t lr = head * p.n_q_tiles + r;
    int nf, np;
    list_counts(p.full_cnt, p.part_cnt, lr, p.list_ld, nf, np);
    int n_hz;  // always 0 here
    const int n = build_steps(p.full_idx + lr * p.list_ld, nf, p.part_idx + lr * p.list_ld, np,
                              lane, steps, [&](int t) {
                                if (t < 0 || t >= nk) return 0;
                                const int vc = clamp_vc(p.valid_count[t]);
                                return vc > kHalf ? 3 : vc > 0 ? 1 : 0;
                              }, n_hz);
    if (lane == 0) step_total = n;
  }

  bf16x8 qf[8], dof[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    qf[s] = as_bf16x8(ld16(p.q + qrow * p.qs + head * p.qh + 16 * s + 8 * hi));
    dof[s] = as_bf16x8(ld16(p.dout + qrow * p.dos + head * p.doh + 16 * s + 8 * hi));
  }
  const float* rec = p.stats + (head * 2 * p.n_q_tiles + 2 * r + (wave >> 1)) * kRecFloats;
  const float lse2 = rec[(32 * wave + li) & 63];
  // -D of this lane's row, the initial accumulator of its dP products
  f32x16 neg_d;
  const float nd = rec[64 + ((32 * wave + li) & 63)];
#pragma unroll
  for (int e = 0; e < 16; ++e) neg_d[e] = nd;
  // A wave whose 32 rows all have dO = 0 and D = 0 (the padding rows of a
  // partial query tile when the caller's gradient comes through the
  // scatter, which drops them): dP - D and dS are exactly 0 there, so its
  // dQ rows are 0 and it only loads and passes the barriers (wave-uniform)
  uint32_t live = nd != 0.f ? 1u : 0u;  // NaN too
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const u32x4 x = __builtin_bit_cast(u32x4, dof[s]);
    live |= ((x[0] | x[1] | x[2] | x[3]) & 0x7FFF7FFFu) != 0 ? 1u : 0u;
  }
  const bool d_zero = __ballot(live != 0) == 0;
  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[dt][e] = 0.f;
  __syncthreads();  // step list and valid counts ready
  const int n_steps = __builtin_amdgcn_readfirstlane(step_total);

  const uint16_t* kbase = p.k + head * p.kh;
  const uint16_t* vbase = p.v + head * p.vh;
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    koff[u] = seg_offset(4 * wave + u, lane, p.ks);
    voff[u] = seg_offset(4 * wave + u, lane, p.vs);
  }
  const Frag f = frag_offsets(lane);
  const float c = p.scale_log2;

  // the step list entry t of a step: (key tile << 1 | half)
  auto load_step = [&](int t, lds_u8* slot) {
    const int64_t row0 = (int64_t)(t >> 1) * kTile + (t & 1) * kHalf;
    const char* kb = reinterpret_cast<const char*>(kbase + row0 * p.ks);
    const char* vb = reinterpret_cast<const char*>(vbase + row0 * p.vs);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      dma16(kb, koff[s], slot + (4 * wave + s) * 1024);
      dma16(vb, voff[s], slot + kHalfBytes + (4 * wave + s) * 1024);
    }
  };
  auto entry = [&](int u) { return __builtin_amdgcn_readfirstlane((int)steps[u]); };
  // One 32-key half kh of a step with `lim` valid keys in it (lim >= 32: all).
  // hook(s) runs between the score products (the walk issues the next
  // step's eight loads there); with a hook the order is written out in the
  // program (a hook that branches ends the scheduling region).
  auto half_step = [&](const lds_u8* slot, int kh, int lim, auto hook) {
    const lds_u8* ks = slot + kh * 32 * 256;
    const lds_u8* vs = slot + kHalfBytes + kh * 32 * 256;
    f32x16 st, dp = neg_d;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.f;
    if constexpr (std::is_same<decltype(hook), NoHook>::value) {
      // S^T and dP^T as two interleaved chains, the reads of k-step s + 2
      // issued before the products of s
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const u32x4 ka = lds16(ks + f.row[s]);
        const u32x4 va = lds16(vs + f.row[s]);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka), qf[s], st, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(va), dof[s], dp, 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int s = 0; s < 6; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    } else {
      // the same reads two k-steps ahead and products, in program order,
      // hook(s) before the reads of k-step s + 2
      u32x4 ka[8], va[8];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        ka[s] = lds16(ks + f.row[s]);
        va[s] = lds16(vs + f.row[s]);
      }
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        hook(s);
        if (s + 2 < 8) {
          ka[s + 2] = lds16(ks + f.row[s + 2]);
          va[s + 2] = lds16(vs + f.row[s + 2]);
        }
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka[s]), qf[s], st, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(va[s]), dof[s], dp, 0, 0, 0);
      }
    }
    float ds[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pr = __builtin_amdgcn_exp2f(fmaf(st[e], c, -lse2));
      ds[e] = pr * dp[e];  // dp holds dP - D
    }
    if (lim < 32) {  // wave-uniform: only the ragged end of a partial tile
      const int l = lim - 4 * hi;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (8 * (e >> 2) + (e & 3) >= l) ds[e] = 0.f;
    }
    u32x4 pk[2];
    pack_b(ds, pk);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag(ks, f, dt, kk), as_bf16x8(pk[kk]),
                                                          acc[dt], 0, 0, 0);
    // issue order: the transposed reads of product i + 2 before product i
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  };
  auto compute = [&](int vch, const lds_u8* slot, auto hook) {
    half_step(slot, 0, vch, hook);
    if (vch > 32) half_step(slot, 1, vch - 32, NoHook{});
  };

  lds_u8* s0 = (lds_u8*)ring[0];
  lds_u8* s1 = (lds_u8*)ring[1];
  // Step u: read the step list (written before the loop) for steps u and
  // u + 1, wait for this wave's loads (the only ones in flight), barrier
  // (every wave's loads of step u are in LDS and every wave is done reading
  // the other slot), issue step u + 1 into the other slot, compute step u.
  // The list reads stay above the barrier, out of the products' schedule.
  auto run = [&](auto zero, int u, lds_u8* cur, lds_u8* nxt) __attribute__((always_inline)) {
    const int t = entry(u);
    const int vc = __builtin_amdgcn_readfirstlane((int)tvc[t >> 1]);
    const int vch = t & 1 ? vc - kHalf : min(vc, kHalf);  // valid keys of the step
    const int tn = u + 1 < n_steps ? entry(u + 1) : 0;
    VEDA_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS read of step u above the barrier
    // step u + 1's loads go out between step u's first score products (in
    // one burst after the barrier, every wave of the CU queues at the load
    // path at once)
    const bool more = u + 1 < n_steps;
    const int64_t row0 = (int64_t)(tn >> 1) * kTile + (tn & 1) * kHalf;
    const char* kb = reinterpret_cast<const char*>(kbase + row0 * p.ks);
    const char* vb = reinterpret_cast<const char*>(vbase + row0 * p.vs);
    auto hook = [&](int s) {
      if (more) {
        if (s < 4) dma16(kb, koff[s], nxt + (4 * wave + s) * 1024);
        else dma16(vb, voff[s - 4], nxt + kHalfBytes + (4 * wave + s - 4) * 1024);
      }
    };
    if constexpr (decltype(zero)::value) {
#pragma unroll
      for (int s = 0; s < 8; ++s) hook(s);
    } else {
      compute(vch, cur, hook);
    }
  };
  // one copy of the walk per kind of wave (the same loads and barriers), so
  // the accumulators stay in one set of registers
  auto walk = [&](auto zero) __attribute__((always_inline)) {
    for (int u = 0; u < n_steps; u += 2) {
      run(zero, u, s0, s1);
      if (u + 1 >= n_steps) break;
      run(zero, u + 1, s1, s0);
    }
  };
  if (n_steps > 0) load_step(entry(0), s0);
  if (d_zero)
    walk(std::true_type{});
  else
    walk(std::false_type{});

  // dQ leaves as whole rows: each wave writes its 32 bf16 rows into its
  // 8 KB of the slot no step reads any more (the last step's is
  // n_steps - 1's; every wave has passed the barrier after step
  // n_steps - 2, which used this one), 16-byte chunk c of row r at
  // c ^ (r % 16), then lane l stores chunk l % 16 of rows 4 i + l / 16:
  // four rows per store instead of 16 bytes of each of 32 rows.
  lds_u8* stage = (lds_u8*)ring[n_steps & 1] + wave * 8192;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x16& a = acc[dt];
      const int e0 = 4 * g;
      const uint32_t w0 = pack_bf16x2(a[e0] * p.scale, a[e0 + 1] * p.scale);
      const uint32_t w1 = pack_bf16x2(a[e0 + 2] * p.scale, a[e0 + 3] * p.scale);
      *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(
          stage + li * 256 + (((4 * dt + g) ^ (li & 15)) << 4) + 8 * hi) = u32x2{w0, w1};
    }
  asm volatile("" ::: "memory");
  const bool row16 = ((reinterpret_cast<uintptr_t>(p.dq) & 15) | ((p.dqs | p.dqh) & 7)) == 0;
  uint16_t* dbase = p.dq + (r * kTile + 32 * wave) * p.dqs + head * p.dqh;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int rr = 4 * i + (lane >> 4), ch = lane & 15;
    const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
        stage + rr * 256 + ((ch ^ (rr & 15)) << 4));
    uint16_t* dst = dbase + rr * p.dqs + 8 * ch;
    if (row16) {
      *reinterpret_cast<u32x4*>(dst) = v;
    } else {  // rows 8-byte aligned only
      *reinterpret_cast<u32x2*>(dst) = u32x2{v[0], v[1]};
      *reinterpret_cast<u32x2*>(dst + 4) = u32x2{v[2], v[3]};
    }
  }
}

// ---------------------------------------------------------------------------
// dK, dV. Workgroup = (head, key tile), 8 waves, one workgroup per CU (two
// waves per SIMD). Every wave runs the whole chain for its own keys and query
// rows, so no product crosses between waves and a step has one barrier (the
// ring's). With v_mfma_f32_16x16x32_bf16 (A[i][k] in lane i + 16 (k / 8) and
// B[k][j] in lane j + 16 (k / 8), element k % 8; D[i][j] in lane
// j + 16 (i / 4), element i % 4) a wave owns 16 keys, K^T and V^T fragments
// in registers (lane n + 16 g: head-dims 32 c + 8 g .. + 7 of key n), and per
// 64-row step NQB blocks of 16 query rows:
//   S = Q K^T, dP - D = dO V^T - D   (4 MFMAs per block each, A = Q / dO rows)
//   P = exp2(S c - lse2), dS = P (dP - D)
//   dV^T += dO^T P, dK^T += Q^T dS   (8 MFMAs per 32 rows each, A = dO^T / Q^T
//                                     from transposed reads)
// Lane n + 16 g holds S, P, dP and dS of rows 16 qb + 4 g + {0..3} of key n.
// That is the B operand of the accumulations when k index e of a 32-row
// chunk stands for row 16 (e / 4) + 4 g + e % 4 (the MFMA sums over k in any
// order); the transposed reads of dO and Q fetch rows in the same order.
// Key tiles with few valid keys spread a step's rows over more waves, which
// add their partial sums at the end:
//   vc > 64: 8 key groups x 4 blocks; 32 < vc <= 64: 4 x 2; vc <= 32: 2 x 1.
//
// The Q and dO slots use their own swizzle (r3..r0 = bits of r mod 16):
//   swzk(r) = 4 (r mod 4) + 2 (r2 xor r3) + r3.
// gfx950 serves a ds_read_b128 in 4 cycles of 16 lanes, lane L in the cycle
// of (L / 32, parity of bits 2-4 of L), and a ds_read_b64 (transposed or
// not) in 2 cycles of 32 lanes (L / 32). With swzk both read patterns of a
// wave put the lanes of each cycle on distinct banks: the row reads (lane
// n + 16 g: row n, chunk 4 cc + g) and the transposed reads (rows
// 4 g + n / 4, chunk 2 db + (n / 2) % 2, half n % 2).

__device__ __forceinline__ int swzk(int r) {
  return ((r & 3) << 2) | ((((r >> 2) ^ (r >> 3)) & 1) << 1) | ((r >> 3) & 1);
}

__device__ __forceinline__ uint32_t seg_offset_k(int seg, int lane, int64_t stride) {
  const int row = 4 * seg + (lane >> 4), pc = lane & 15;
  return (uint32_t)((row * stride + ((pc ^ swzk(row)) << 3)) * 2);
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__global__ void __launch_bounds__(kDkvThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) dkv_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[2][kSlot + kRecBytes];
  __shared__ uint16_t steps[2 * kMaxTiles];
  __shared__ int32_t step_total, step_hz;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  int64_t head, j;
  front_first(blockIdx.x, p.n_heads, p.n_k_tiles, p.front, head, j);
  const int vc = __builtin_amdgcn_readfirstlane(clamp_vc(p.valid_count[j]));
  const int nq = (int)p.n_q_tiles;

  if (wave == 0) {
    const int64_t lr = head * p.n_k_tiles + j;
    int nf, np;
    list_counts(p.full_cnt_t, p.part_cnt_t, lr, p.list_ld_t, nf, np);
    // A 64-row half whose rows all have dO = 0 and D = 0 (the padding rows
    // of a partial query tile when the caller's gradient comes through the
    // scatter, which drops them) adds exactly zero to dK and dV: no step. One
    // whose rows 32 .. 63 alone have them is an upper-zero step: only its
    // first 32 rows are computed, in a second walk after the others.
    const float* zrec = p.stats + head * 2 * p.n_q_tiles * kRecFloats + kZeroFlag;
    int n_hz;
    const int cnt = build_steps(p.full_idx_t + lr * p.list_ld_t, nf,
                                p.part_idx_t + lr * p.list_ld_t, np, lane, steps, [&](int t) {
                                  if (vc <= 0 || t < 0 || t >= nq) return 0;
                                  const float* r0 = zrec + (2 * t) * kRecFloats;
                                  const float* r1 = r0 + kRecFloats;
                                  constexpr int h = kHiZeroFlag - kZeroFlag;
                                  return (r0[0] != 0.f ? 0 : 1) | (r1[0] != 0.f ? 0 : 2) |
                                         (r0[h] != 0.f ? 4 : 0) | (r1[h] != 0.f ? 8 : 0);
                                }, n_hz);
    if (lane == 0) {
      step_total = cnt;
      step_hz = n_hz;
    }
  }
  f32x4 acc_v[8], acc_k[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) acc_v[db] = acc_k[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  // steps 0 .. n_full - 1 are the others, n_full .. n_steps - 1 upper-zero
  const int n_full = __builtin_amdgcn_readfirstlane(step_total);
  const int n_steps = n_full + __builtin_amdgcn_readfirstlane(step_hz);
  auto entry = [&](int u) {
    return __builtin_amdgcn_readfirstlane(
        (int)steps[u < n_full ? u : 2 * kMaxTiles - 1 - (u - n_full)]);
  };

  const uint16_t* qbase = p.q + head * p.qh;
  const uint16_t* dbase = p.dout + head * p.doh;
  uint32_t qoff[2], doff[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    qoff[u] = seg_offset_k(2 * wave + u, lane, p.qs);
    doff[u] = seg_offset_k(2 * wave + u, lane, p.dos);
  }
  const float c = p.scale_log2;

  auto load_step = [&](int u, lds_u8* slot) {
    const int t = entry(u);
    const int64_t row0 = (int64_t)(t >> 1) * kTile + (t & 1) * kHalf;
    const char* qb = reinterpret_cast<const char*>(qbase + row0 * p.qs);
    const char* db = reinterpret_cast<const char*>(dbase + row0 * p.dos);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      dma16(qb, qoff[s], slot + (2 * wave + s) * 1024);
      dma16(db, doff[s], slot + kHalfBytes + (2 * wave + s) * 1024);
    }
    if (wave == 0) {
      const float* rec = p.stats + (head * 2 * p.n_q_tiles + t) * kRecFloats;
      dma16(reinterpret_cast<const char*>(rec), (uint32_t)(lane * 16), slot + kSlot);
    }
  };

  lds_u8* s0 = (lds_u8*)ring[0];
  lds_u8* s1 = (lds_u8*)ring[1];
  // NQB query blocks per wave and step; FULL: every key of the tile valid.
  auto body = [&](auto nqb, auto full) __attribute__((always_inline)) {
    constexpr int NQB = decltype(nqb)::value;
    constexpr bool FULL = decltype(full)::value;
    constexpr int NKG = 2 * NQB;                           // key groups of 16
    const int kgrp = wave % NKG, qb0 = (wave / NKG) * NQB;  // this wave's keys and first block
    const int key = 16 * kgrp + n;
    const bool key_ok = key < vc;
    const bool live = 16 * kgrp < vc;
    const int64_t krow = j * kTile + key;
    u32x4 kf[4], vf[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      kf[cc] = ld16(p.k + krow * p.ks + head * p.kh + 32 * cc + 8 * g);
      vf[cc] = ld16(p.v + krow * p.vs + head * p.vh + 32 * cc + 8 * g);
    }
    // LDS byte offsets inside a slot: row reads (row 16 qb + n, chunk 4 cc + g)
    // and transposed reads (rows 16 qb + 4 g + n / 4 (+ 16), head-dims
    // 16 db + 4 (n % 4) .. + 3, i.e. chunk 2 db + (n / 2) % 2, half n % 2)
    uint32_t arow[4], tro[8];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) arow[cc] = qb0 * 4096 + n * 256 + (((4 * cc + g) ^ swzk(n)) << 4);
    const int rt = 4 * g + (n >> 2);
#pragma unroll
    for (int db = 0; db < 8; ++db)
      tro[db] = (16 * qb0 + rt) * 256 + (((2 * db + ((n >> 1) & 1)) ^ swzk(rt)) << 4) + 8 * (n & 1);
    const uint32_t roff = 4 * (16 * qb0 + 4 * g);  // the record's lse2 of the lane's rows

    // NB (<= NQB) blocks of this wave's rows: NQB, or 2 (blocks 0, 1: rows
    // 0 .. 31) in an upper-zero step of a wave of blocks 0 .. 3
    auto compute = [&](auto nb, const lds_u8* slot) __attribute__((always_inline)) {
      constexpr int NB = decltype(nb)::value;
      const lds_u8* qs = slot;
      const lds_u8* ds = slot + kHalfBytes;
      const lds_u8* rec = slot + kSlot;
      f32x4 s[NB], dp[NB], lse[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[i] = *reinterpret_cast<const lds_f32x4*>(rec + 256 + roff + 64 * i);  // -D
        lse[i] = *reinterpret_cast<const lds_f32x4*>(rec + roff + 64 * i);
      }
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int i = 0; i < NB; ++i)
          s[i] = mfma16(lds16(qs + i * 4096 + arow[cc]), kf[cc], s[i]);
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int i = 0; i < NB; ++i)
          dp[i] = mfma16(lds16(ds + i * 4096 + arow[cc]), vf[cc], dp[i]);
      // issue order: the record reads, then each row read four products
      // ahead of its product
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * NB + 4, 0);
#pragma unroll
      for (int x = 0; x < 8 * NB - 4; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      uint32_t pp[NB][2], pd[NB][2];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const f32x4 l4 = lse[i];
        float pr[4], dv[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float x = __builtin_amdgcn_exp2f(fmaf(s[i][m], c, -l4[m]));
          pr[m] = FULL || key_ok ? x : 0.f;
          const float y = pr[m] * dp[i][m];  // dp holds dP - D
          dv[m] = FULL || key_ok ? y : 0.f;
        }
        pp[i][0] = pack_bf16x2(pr[0], pr[1]);
        pp[i][1] = pack_bf16x2(pr[2], pr[3]);
        pd[i][0] = pack_bf16x2(dv[0], dv[1]);
        pd[i][1] = pack_bf16x2(dv[2], dv[3]);
      }
      constexpr int NC = NB == 1 ? 1 : NB / 2;  // 32-row chunks
#pragma unroll
      for (int qc = 0; qc < NC; ++qc) {
        u32x4 bp, bd;
        if constexpr (NB == 1) {
          bp = u32x4{pp[0][0], pp[0][1], 0u, 0u};
          bd = u32x4{pd[0][0], pd[0][1], 0u, 0u};
        } else {
          bp = u32x4{pp[2 * qc][0], pp[2 * qc][1], pp[2 * qc + 1][0], pp[2 * qc + 1][1]};
          bd = u32x4{pd[2 * qc][0], pd[2 * qc][1], pd[2 * qc + 1][0], pd[2 * qc + 1][1]};
        }
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          const u32x2 zero2 = {0u, 0u};
          const lds_u8* da = ds + qc * 8192 + tro[db];
          const lds_u8* qa = qs + qc * 8192 + tro[db];
          const u32x2 dlo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)da));
          const u32x2 dhi = NB == 1 ? zero2
                                     : __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                                     (lds_i16x4*)(da + 4096)));
          acc_v[db] = mfma16(u32x4{dlo[0], dlo[1], dhi[0], dhi[1]}, bp, acc_v[db]);
          const u32x2 qlo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)qa));
          const u32x2 qhi = NB == 1 ? zero2
                                     : __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                                     (lds_i16x4*)(qa + 4096)));
          acc_k[db] = mfma16(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]}, bd, acc_k[db]);
        }
        // issue order: the reads of head-dim block db + 1 before the products of db
        constexpr int R = NB == 1 ? 2 : 4;
        __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
#pragma unroll
        for (int db = 1; db < 8; ++db) {
          __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      }
    };
    // Step u: wait for this wave's loads (the only ones in flight), barrier
    // (every wave's loads of step u are in LDS and every wave is done reading
    // the other slot), issue step u + 1 into the other slot, compute step u.
    // The others first, then the upper-zero steps (hz), each walk with its
    // own code, so the accumulators stay in one set of registers.
    auto run = [&](auto hz, int u, lds_u8* cur, lds_u8* nxt) __attribute__((always_inline)) {
      VEDA_WAIT_VM(0);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (u + 1 < n_steps) load_step(u + 1, nxt);
      if (live) {
        if constexpr (!decltype(hz)::value)
          compute(std::integral_constant<int, NQB>{}, cur);
        else if constexpr (NQB == 4)
          compute(std::integral_constant<int, 2>{}, cur);
        else if (qb0 < 2)  // a wave of rows 32 .. 63 has nothing to add
          compute(std::integral_constant<int, NQB>{}, cur);
      }
    };
    auto walk = [&](auto hz, int u, int end) __attribute__((always_inline)) {
      if (u < end && (u & 1)) run(hz, u++, s1, s0);
      for (; u < end; u += 2) {
        run(hz, u, s0, s1);
        if (u + 1 >= end) break;
        run(hz, u + 1, s1, s0);
      }
    };
    if (n_steps > 0) load_step(0, s0);
    walk(std::false_type{}, 0, n_full);
    walk(std::true_type{}, n_full, n_steps);
    if constexpr (NQB < 4) {
      // the waves of key group kgrp (kgrp + NKG x part) hand their partial
      // sums to wave kgrp through the ring (free now); dV first, then dK
      lds_f32x4* red = reinterpret_cast<lds_f32x4*>(s0) + lane;
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
        f32x4(&a)[8] = pass == 0 ? acc_v : acc_k;
        __syncthreads();
        if (wave >= NKG) {
#pragma unroll
          for (int db = 0; db < 8; ++db) {
            red[((wave - NKG) * 8 + db) * 64] = a[db];
            a[db] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
        __syncthreads();
        if (wave < NKG) {
#pragma unroll
          for (int part = 1; part < 4 / NQB; ++part)
#pragma unroll
            for (int db = 0; db < 8; ++db) a[db] += red[((wave + NKG * (part - 1)) * 8 + db) * 64];
        }
      }
    }
  };
  using B4 = std::integral_constant<int, 4>;
  using B2 = std::integral_constant<int, 2>;
  using B1 = std::integral_constant<int, 1>;
  if (vc == kTile)
    body(B4{}, std::true_type{});
  else if (vc > 64)
    body(B4{}, std::false_type{});
  else if (vc > 32)
    body(B2{}, std::false_type{});
  else
    body(B1{}, std::false_type{});

  // wave w writes rows 16 w .. + 15 of the tile (zeros past the computed key
  // groups: those keys are padding), head-dims 16 db + 4 g .. + 3
  const int64_t orow = j * kTile + 16 * wave + n;
  uint16_t* vrow = p.dv + orow * p.dvs + head * p.dvh;
  uint16_t* krw = p.dk + orow * p.dks + head * p.dkh;
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    const f32x4 av = acc_v[db], ak = acc_k[db];
    *reinterpret_cast<u32x2*>(vrow + 16 * db + 4 * g) =
        u32x2{pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3])};
    *reinterpret_cast<u32x2*>(krw + 16 * db + 4 * g) =
        u32x2{pack_bf16x2(ak[0] * p.scale, ak[1] * p.scale), pack_bf16x2(ak[2] * p.scale, ak[3] * p.scale)};
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" int veda_block_sparse_bwd(
    const void* q, int64_t q_stride_s, int64_t q_stride_h, const void* k, int64_t k_stride_s,
    int64_t k_stride_h, const void* v, int64_t v_stride_s, int64_t v_stride_h, const void* out,
    int64_t o_stride_s, int64_t o_stride_h, const void* dout, int64_t do_stride_s,
    int64_t do_stride_h, const float* lse, int64_t lse_stride_h, int64_t lse_stride_s,
    const float* dlse, int64_t dlse_stride_h, int64_t dlse_stride_s, int64_t n_heads,
    int64_t head_dim, int64_t n_q_tiles, int64_t n_k_tiles,
    const int32_t* full_cnt, const int32_t* full_idx, const int32_t* part_cnt,
    const int32_t* part_idx, int64_t list_ld, const int32_t* full_cnt_t,
    const int32_t* full_idx_t, const int32_t* part_cnt_t, const int32_t* part_idx_t,
    int64_t list_ld_t, const int32_t* valid_count, float scale, void* dq, int64_t dq_stride_s,
    int64_t dq_stride_h, void* dk, int64_t dk_stride_s, int64_t dk_stride_h, void* dv,
    int64_t dv_stride_s, int64_t dv_stride_h, void* workspace, int64_t workspace_bytes,
    int64_t front_tiles, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_sparse_bwd: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0 && n_k_tiles >= 0, "block_sparse_bwd: negative size");
  VEDA_REQUIRE(n_q_tiles <= kMaxTiles && n_k_tiles <= kMaxTiles,
               "block_sparse_bwd: at most %d query and key tiles, got %lld and %lld", kMaxTiles,
               (long long)n_q_tiles, (long long)n_k_tiles);
  VEDA_REQUIRE(list_ld >= n_k_tiles && list_ld_t >= n_q_tiles,
               "block_sparse_bwd: list rows must hold n_k_tiles (forward) and n_q_tiles "
               "(transposed) entries");
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && aligned16(dout) &&
                   q_stride_s % 8 == 0 && q_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   k_stride_h % 8 == 0 && v_stride_s % 8 == 0 && v_stride_h % 8 == 0 &&
                   o_stride_s % 8 == 0 && o_stride_h % 8 == 0 && do_stride_s % 8 == 0 &&
                   do_stride_h % 8 == 0,
               "block_sparse_bwd: q, k, v, out, dout rows must be 16-byte aligned");
  VEDA_REQUIRE(aligned8(dq) && aligned8(dk) && aligned8(dv) && dq_stride_s % 4 == 0 &&
                   dq_stride_h % 4 == 0 && dk_stride_s % 4 == 0 && dk_stride_h % 4 == 0 &&
                   dv_stride_s % 4 == 0 && dv_stride_h % 4 == 0,
               "block_sparse_bwd: dq, dk, dv rows must be 8-byte aligned");
  // the LDS loads address a 64-row step with 32-bit byte offsets
  VEDA_REQUIRE(q_stride_s < (1 << 24) && k_stride_s < (1 << 24) && v_stride_s < (1 << 24) &&
                   do_stride_s < (1 << 24),
               "block_sparse_bwd: row stride too large");
  VEDA_REQUIRE(front_tiles >= 0 && front_tiles <= n_q_tiles && front_tiles <= n_k_tiles,
               "block_sparse_bwd: front_tiles %lld outside [0, min(n_q_tiles, n_k_tiles)]",
               (long long)front_tiles);
  const int64_t need = n_heads * 2 * n_q_tiles * kRecBytes;
  VEDA_REQUIRE(aligned16(workspace) && workspace_bytes >= need,
               "block_sparse_bwd: workspace needs %lld bytes (16-byte aligned), got %lld",
               (long long)need, (long long)workspace_bytes);
  BwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(out);
  p.dout = static_cast<const uint16_t*>(dout);
  p.qs = q_stride_s; p.qh = q_stride_h;
  p.ks = k_stride_s; p.kh = k_stride_h;
  p.vs = v_stride_s; p.vh = v_stride_h;
  p.os = o_stride_s; p.oh = o_stride_h;
  p.dos = do_stride_s; p.doh = do_stride_h;
  p.lse = lse; p.lse_sh = lse_stride_h; p.lse_ss = lse_stride_s;
  p.dlse = dlse; p.dlse_sh = dlse_stride_h; p.dlse_ss = dlse_stride_s;
  p.n_heads = n_heads; p.n_q_tiles = n_q_tiles; p.n_k_tiles = n_k_tiles;
  p.full_cnt = full_cnt; p.full_idx = full_idx; p.part_cnt = part_cnt; p.part_idx = part_idx;
  p.list_ld = list_ld;
  p.full_cnt_t = full_cnt_t; p.full_idx_t = full_idx_t;
  p.part_cnt_t = part_cnt_t; p.part_idx_t = part_idx_t;
  p.list_ld_t = list_ld_t;
  p.valid_count = valid_count;
  p.scale = scale;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.stats = static_cast<float*>(workspace);
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.dqs = dq_stride_s; p.dqh = dq_stride_h;
  p.dks = dk_stride_s; p.dkh = dk_stride_h;
  p.dvs = dv_stride_s; p.dvh = dv_stride_h;
  p.front = front_tiles;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t q_items = n_heads * n_q_tiles, k_items = n_heads * n_k_tiles;
  if (q_items > 0) {
    bwd_stats_kernel<<<(unsigned)(2 * q_items), 256, 0, s>>>(p);
    if (int rc = check_launch("veda_block_sparse_bwd (stats)")) return rc;
    dq_kernel<<<(unsigned)q_items, kDqThreads, 0, s>>>(p);
    if (int rc = check_launch("veda_block_sparse_bwd (dq)")) return rc;
  }
  if (k_items > 0) {
    dkv_kernel<<<(unsigned)k_items, kDkvThreads, 0, s>>>(p);
    return check_launch("veda_block_sparse_bwd (dk, dv)");
  }
  return VEDA_OK;
}

// ---------------------------------------------------------------------------
// The backward without allocation: the per-row statistics go to a
// file-scope device array instead of a caller workspace, for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).
//
// In host code `scratch` names a host-side stand-in, not a device address:
// every use goes through the address hipGetSymbolAddress returns for the
// device, looked up once per device (on the first call with that device
// current) and kept in g_scratch_addr. Each device holds its own copy of the
// array for the life of the process. Nothing in it must start at zero: the
// statistics kernel writes every record the gradient kernels read.

namespace veda {
namespace {

constexpr int64_t kScratchBytes = int64_t(64) << 20;  // 64 MiB
constexpr int kScratchDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_addr[kScratchDevices] = {};

// The device address of `scratch` on the current device, which must be the
// device of `stream`.
int scratch_address(void* stream, void** addr) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("block_sparse_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(err));
    return VEDA_ELAUNCH;
  }
  if (stream != nullptr) {
    int sdev = -1;
    err = hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev);
    if (err != hipSuccess) {
      set_error("block_sparse_bwd_noalloc: hipStreamGetDevice failed: %s",
                hipGetErrorString(err));
      return VEDA_ELAUNCH;
    }
    VEDA_REQUIRE(sdev == dev,
                 "block_sparse_bwd_noalloc: the stream belongs to device %d, but device %d is "
                 "current",
                 sdev, dev);
  }
  VEDA_REQUIRE(dev >= 0 && dev < kScratchDevices,
               "block_sparse_bwd_noalloc: device %d outside [0, %d)", dev, kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      set_error("block_sparse_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(err));
      return VEDA_ELAUNCH;
    }
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return VEDA_OK;
}

}  // namespace
}  // namespace veda

extern "C" int veda_block_sparse_bwd_noalloc(
    const void* q, int64_t q_stride_s, int64_t q_stride_h, const void* k, int64_t k_stride_s,
    int64_t k_stride_h, const void* v, int64_t v_stride_s, int64_t v_stride_h, const void* out,
    int64_t o_stride_s, int64_t o_stride_h, const void* dout, int64_t do_stride_s,
    int64_t do_stride_h, const float* lse, int64_t lse_stride_h, int64_t lse_stride_s,
    const float* dlse, int64_t dlse_stride_h, int64_t dlse_stride_s, int64_t n_heads,
    int64_t head_dim, int64_t n_q_tiles, int64_t n_k_tiles,
    const int32_t* full_cnt, const int32_t* full_idx, const int32_t* part_cnt,
    const int32_t* part_idx, int64_t list_ld, const int32_t* full_cnt_t,
    const int32_t* full_idx_t, const int32_t* part_cnt_t, const int32_t* part_idx_t,
    int64_t list_ld_t, const int32_t* valid_count, float scale, void* dq, int64_t dq_stride_s,
    int64_t dq_stride_h, void* dk, int64_t dk_stride_s, int64_t dk_stride_h, void* dv,
    int64_t dv_stride_s, int64_t dv_stride_h, int64_t front_tiles, void* stream) {
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0 && n_q_tiles <= kMaxTiles,
               "block_sparse_bwd_noalloc: bad sizes (%lld heads, %lld query tiles)",
               (long long)n_heads, (long long)n_q_tiles);
  const int64_t need = n_heads * 2 * n_q_tiles * kRecBytes;
  VEDA_REQUIRE(need <= kScratchBytes,
               "block_sparse_bwd_noalloc: %lld heads x %lld query tiles need %lld bytes of "
               "statistics, more than its %lld-byte scratch; split the heads or call "
               "veda_block_sparse_bwd with a workspace",
               (long long)n_heads, (long long)n_q_tiles, (long long)need,
               (long long)kScratchBytes);
  void* work = nullptr;
  if (int rc = scratch_address(stream, &work)) return rc;
  return veda_block_sparse_bwd(
      q, q_stride_s, q_stride_h, k, k_stride_s, k_stride_h, v, v_stride_s, v_stride_h, out,
      o_stride_s, o_stride_h, dout, do_stride_s, do_stride_h, lse, lse_stride_h, lse_stride_s,
      dlse, dlse_stride_h, dlse_stride_s, n_heads, head_dim, n_q_tiles, n_k_tiles, full_cnt,
      full_idx, part_cnt, part_idx, list_ld, full_cnt_t, full_idx_t, part_cnt_t, part_idx_t,
      list_ld_t, valid_count, scale, dq, dq_stride_s, dq_stride_h, dk, dk_stride_s, dk_stride_h,
      dv, dv_stride_s, dv_stride_h, work, kScratchBytes, front_tiles, stream);
}
