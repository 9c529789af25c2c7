// Block-sparse flash-attention forward for gfx950 (head_dim 128, bf16 in,
// fp32 accumulate), and the dense forward built from the same kernel.
//
// Workgroup = one (head, 128-row query tile), 8 waves, 1 workgroup per CU:
//   wave w: query group qg = w % 4 (32 query rows), key half kh = w / 4
//   (keys [64 kh, 64 kh + 64) of every 128-key block).
// Two waves share each SIMD, so one wave's softmax overlaps the other's
// MFMAs. The two key halves keep separate online-softmax states and are
// merged through LDS at the end.
//
// Scores are computed transposed, S^T = K Q^T with v_mfma_f32_32x32x16_bf16
// (A = K rows from LDS, B = Q^T held in registers), so every lane owns ONE
// query row and 16 of the keys of a 32-key sub-tile: the row max needs one
// cross-half lane swap, the rescale of O is a per-lane scalar, and P^T feeds
// the P.V product straight from the accumulator registers:
//   O^T[d, i] += V^T[d, key] P^T[key, i]   (A = V^T, B = P^T).
// The MFMA contracts over k, so the order of the 16 keys of one k-step is
// free: lane half h supplies keys 16s + 4h + {0..3, 8..11}, the order in
// which the accumulator registers hold P^T.
//
// K and V tiles go from HBM straight into LDS (global_load_lds_dwordx4: lane
// l of a wave writes bytes [16 l, 16 l + 16) of a 1 KB segment), two stages,
// the next block's loads in flight while the current block is computed; no
// register staging and no transposing stores. Both tiles keep their natural
// [key][head_dim] row layout with the 16-byte chunks of row r permuted:
//   K: chunk c at position c ^ (r & 15)   -> the 16-byte K fragment reads of
//      32 consecutive rows are conflict-free;
//   V: chunk c at position c ^ 4 (r & 3)  -> the V^T fragments, assembled by
//      two ds_read_b64_tr_b16 (lane i of a 16-lane group receives element
//      (i mod 4) of source lane 4 j + i / 4, j = 0..3), are conflict-free.
// The walk over kept blocks is unrolled by two over two distinct LDS arrays,
// so the DMA into one stage provably does not alias the reads of the other.

#include "veda_common.h"

namespace veda {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 512;
constexpr int kTileBytes = kTile * kD * 2;       // 32 KB: one K or V tile
constexpr int kStageBytes = 2 * kTileBytes;      // K + V
constexpr int kMaxBlocks = 2048;                 // key tiles per row (FA4's cap)
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.f;             // log2 units

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t qs, qh, ks, kh, vs, vh;
  int64_t n_heads, n_q_tiles, n_k_tiles;
  const int32_t* full_cnt;
  const int32_t* full_idx;
  const int32_t* part_cnt;
  const int32_t* part_idx;
  int64_t list_ld;
  const int32_t* valid_count;
  int64_t used;      // dense mode: real rows; sparse mode: unused
  int64_t kv_rows;   // rows of k / v that may be read (>= 1 when any block runs)
  int64_t q_rows;    // rows of q / out / lse that exist
  float scale_log2;  // softmax scale * log2(e)
  uint16_t* out;
  int64_t os, oh;
  float* lse;
  int64_t lse_sh, lse_ss;
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// max / sum with the lane 32 positions away (v_permlane32_swap leaves {own,
// partner} in the two results of every lane, in either order).
__device__ __forceinline__ float half_swap_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Issues the HBM -> LDS loads of block j into one stage: wave w fills K and
// V segments 4w .. 4w+3 (rows 16w .. 16w+15); rows past kv_rows are clamped
// (a clamped row only ever feeds masked keys).
__device__ __forceinline__ void issue_stage(const FwdParams& p, int64_t head, int64_t j, int wave,
                                            int lane, lds_u8* stage) {
  const int64_t row0 = j * kTile;
  const int64_t rem = p.kv_rows - 1 - row0;
  const int last = rem < kTile - 1 ? (int)rem : kTile - 1;
  const uint16_t* kbase = p.k + head * p.kh + row0 * p.ks;
  const uint16_t* vbase = p.v + head * p.vh + row0 * p.vs;
  const int ks = (int)p.ks, vs = (int)p.vs;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int seg = 4 * wave + u;
    const int row = 4 * seg + (lane >> 4), pc = lane & 15;
    const int src = min(row, last);
    __builtin_amdgcn_global_load_lds(kbase + (src * ks + ((pc ^ (row & 15)) << 3)),
                                     (lds_void*)(stage + seg * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(vbase + (src * vs + ((pc ^ ((row & 3) << 2)) << 3)),
                                     (lds_void*)(stage + kTileBytes + seg * 1024), 16, 0, 0);
  }
}

struct Walk {
  const int32_t* j;   // LDS: key tile of every step
  const int32_t* vc;  // LDS: valid keys of every step
};

struct WaveState {
  bf16x8 qf[8];
  f32x16 o[4];
  float m_run, l_run;
};

// One block (128 keys) of the online softmax for this wave's 32 rows and 64
// keys, reading K and V from `stage`.
__device__ __forceinline__ void attend_block(const FwdParams& p, const lds_u8* stage, int vc,
                                             int kh, int li, int hi, int lane, WaveState& w) {
  const lds_u8* kb = stage;
  const lds_u8* vb = stage + kTileBytes;
  // S^T: two 32-key sub-tiles, accumulator chains alternating.
  f32x16 sacc[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    sacc[0][e] = 0.f;
    sacc[1][e] = 0.f;
  }
  {
    // row 64 kh + 32 t2 + li, logical chunk 2 s + hi at (2 s + hi) ^ (li & 15)
    const int x = (hi ^ (li & 15)) << 4;
    const lds_u8* r0 = kb + (64 * kh + li) * 256;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int off = x ^ (s << 5);
      const u32x4 a0 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(r0 + off);
      const u32x4 a1 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(r0 + 32 * 256 + off);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a0), w.qf[s], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a1), w.qf[s], sacc[1], 0, 0, 0);
    }
  }
  // Register e of sub-tile t2 is key 64 kh + 32 t2 + 8 (e / 4) + 4 hi + e % 4.
  if (vc < kTile) {
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = 64 * kh + 32 * t2 + 8 * (e >> 2) + 4 * hi + (e & 3);
        if (key >= vc) sacc[t2][e] = -INFINITY;
      }
  }
  // Online softmax in the log2 domain: p = exp2(s * c - m). The reference max
  // m rises only when a row's max passes it by more than kRescaleSlack (p then
  // stays <= 2^kRescaleSlack, exact in fp32 and bf16), so the O rescale is
  // skipped for most blocks; numerator and denominator share m.
  float mloc = -INFINITY;
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, sacc[t2][e]);
  mloc = half_swap_max(mloc) * p.scale_log2;
  const float m_new = mloc > w.m_run + kRescaleSlack ? mloc : w.m_run;
  const float m_use = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_use);
  w.m_run = m_new;
  float lsum = 0.f;
  u32x4 pk[2][2];
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float a = __builtin_amdgcn_exp2f(fmaf(sacc[t2][8 * kk + 2 * m], p.scale_log2, -m_use));
        const float b = __builtin_amdgcn_exp2f(fmaf(sacc[t2][8 * kk + 2 * m + 1], p.scale_log2, -m_use));
        lsum += a + b;
        pk[t2][kk][m] = pack_bf16x2(a, b);
      }
  w.l_run = w.l_run * alpha + lsum;
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) w.o[dt][e] *= alpha;
  }
  // O^T += V^T P^T over the wave's four 16-key groups. Fragment of lane
  // (16-lane group g = (hi, dh), i): two transposed reads of rows
  // 16 s + 4 hi + i / 4 (+ 8), head-dims 32 dt + 16 dh + 4 (i % 4) .. + 3.
  const int i16 = lane & 15, q4 = i16 >> 2, dh = (lane >> 4) & 1;
  const int vbase = (4 * hi + q4) * 256 + (((2 * dh + ((i16 >> 1) & 1)) << 4) | (q4 << 6)) +
                    (i16 & 1) * 8;
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int s = 4 * kh + 2 * t2 + kk;
      const bf16x8 b = as_bf16x8(pk[t2][kk]);
      const lds_u8* vs = vb + s * 16 * 256;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int off = vbase ^ (dt << 6);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vs + off));
        const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vs + 8 * 256 + off));
        typedef short i16x8 __attribute__((ext_vector_type(8)));
        const i16x8 a = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
        w.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), b, w.o[dt],
                                                         0, 0, 0);
      }
    }
}

template <bool DENSE>
__global__ void __launch_bounds__(kThreads) fwd_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[kStageBytes];
  __shared__ int32_t walk_j[kMaxBlocks];
  __shared__ int32_t walk_vc[kMaxBlocks];
  lds_u8* st0 = (lds_u8*)stage0;
  lds_u8* st1 = (lds_u8*)stage1;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int qg = wave & 3, kh = wave >> 2;
  const int li = lane & 31, hi = lane >> 5;
  const int64_t item = blockIdx.x;
  const int64_t head = item / p.n_q_tiles;
  const int64_t r = item % p.n_q_tiles;
  const int64_t qrow = r * kTile + 32 * qg + li;

  int nf, nb;
  if (DENSE) {
    nf = 0;
    nb = (int)((p.used + kTile - 1) / kTile);
  } else {
    const int64_t li_ = head * p.n_q_tiles + r;
    const int ld = (int)p.list_ld;
    nf = min(max(p.full_cnt[li_], 0), ld);
    nb = min(nf + min(max(p.part_cnt[li_], 0), ld), kMaxBlocks);
    // The block walk -- key tile and valid key count of every step, full
    // list first -- goes to LDS once, so the loop reads no list or count
    // from global memory (a vector load behind the in-flight K / V loads
    // would make its wait a wait for them). An entry outside [0, n_k_tiles)
    // keeps no key.
    const int32_t* fl = p.full_idx + li_ * p.list_ld;
    const int32_t* pl = p.part_idx + li_ * p.list_ld;
    for (int i = tid; i < nb; i += kThreads) {
      int64_t j = i < nf ? fl[i] : pl[i - nf];
      int vc;
      if (j < 0 || j >= p.n_k_tiles) {
        j = 0;
        vc = 0;
      } else {
        vc = i < nf ? kTile : p.valid_count[j];
      }
      walk_j[i] = (int32_t)j;
      walk_vc[i] = vc;
    }
  }

  WaveState w;
  // Q^T fragments: lane (li, hi) holds q[qrow, 16 s + 8 hi + 0..7].
  const bool q_ok = DENSE ? (qrow < p.used) : true;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    u32x4 v = q_ok ? ld16(p.q + qrow * p.qs + head * p.qh + 16 * s + 8 * hi) : u32x4{0, 0, 0, 0};
    w.qf[s] = as_bf16x8(v);
  }
  // Consume the Q loads here: otherwise the wait-count pass carries them into
  // the loop and waits on the in-flight K/V loads before every MFMA.
#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" : : "v"(w.qf[s]));
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) w.o[dt][e] = 0.f;
  w.m_run = -INFINITY;
  w.l_run = 0.f;
  __syncthreads();  // walk ready

  auto step_block = [&](int t) -> int64_t {
    return DENSE ? t : __builtin_amdgcn_readfirstlane(walk_j[t]);
  };
  auto step_count = [&](int t) -> int {
    if (DENSE) {
      const int64_t rem = p.used - (int64_t)t * kTile;
      return rem < kTile ? (int)rem : kTile;
    }
    return __builtin_amdgcn_readfirstlane(walk_vc[t]);
  };
  if (nb > 0) issue_stage(p, head, step_block(0), wave, lane, st0);
  for (int t = 0; t < nb; t += 2) {
    // even step: compute stage 0 while stage 1 fills
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 1 < nb) issue_stage(p, head, step_block(t + 1), wave, lane, st1);
    attend_block(p, st0, step_count(t), kh, li, hi, lane, w);
    if (t + 1 >= nb) break;
    // odd step: compute stage 1 while stage 0 fills
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 2 < nb) issue_stage(p, head, step_block(t + 2), wave, lane, st0);
    attend_block(p, st1, step_count(t + 1), kh, li, hi, lane, w);
  }
  __syncthreads();  // every wave is done reading both stages

  // Merge the two key halves: kh = 1 hands (m, l, O) to kh = 0 through LDS.
  w.l_run = half_swap_sum(w.l_run);
  float* red = reinterpret_cast<float*>(stage0);  // [qg][64 regs][64 lanes] = 64 KB
  float* ml = reinterpret_cast<float*>(stage1);   // [qg][2][32]
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[(qg * 64 + dt * 16 + e) * 64 + lane] = w.o[dt][e];
    if (hi == 0) {
      ml[qg * 64 + li] = w.m_run;
      ml[qg * 64 + 32 + li] = w.l_run;
    }
  }
  __syncthreads();
  if (kh == 1) return;
  const float m1 = ml[qg * 64 + li], l1 = ml[qg * 64 + 32 + li];
  const float m = fmaxf(w.m_run, m1);
  const float mu = m == -INFINITY ? 0.f : m;
  const float a0 = __builtin_amdgcn_exp2f(w.m_run - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
  const float l = w.l_run * a0 + l1 * a1;
  const bool row_real = DENSE ? (qrow < p.used) : true;
  const float inv = (l > 0.f && row_real) ? 1.f / l : 0.f;
  if (qrow >= p.q_rows) return;  // dense mode: rows past seq_len do not exist
  uint16_t* orow = p.out + qrow * p.os + head * p.oh;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v4[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int e = 4 * g + rr;
        const float o1 = red[(qg * 64 + dt * 16 + e) * 64 + lane];
        v4[rr] = (w.o[dt][e] * a0 + o1 * a1) * inv;
      }
      const int d = 32 * dt + 8 * g + 4 * hi;
      uint32_t w0 = pack_bf16x2(v4[0], v4[1]), w1 = pack_bf16x2(v4[2], v4[3]);
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2*>(orow + d) = u32x2{w0, w1};
    }
  if (p.lse != nullptr && hi == 0) {
    float lse;
    if (!row_real) lse = 0.f;
    else lse = l > 0.f ? (m + __log2f(l)) * kLn2 : -INFINITY;
    p.lse[head * p.lse_sh + qrow * p.lse_ss] = lse;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" int veda_block_sparse_fwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                                     const void* k, int64_t k_stride_s, int64_t k_stride_h,
                                     const void* v, int64_t v_stride_s, int64_t v_stride_h,
                                     int64_t n_heads, int64_t head_dim, int64_t n_q_tiles,
                                     int64_t n_k_tiles, const int32_t* full_cnt,
                                     const int32_t* full_idx, const int32_t* part_cnt,
                                     const int32_t* part_idx, int64_t list_ld,
                                     const int32_t* valid_count, float scale, void* out,
                                     int64_t o_stride_s, int64_t o_stride_h, float* lse,
                                     int64_t lse_stride_h, int64_t lse_stride_s, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_sparse_fwd: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0 && n_k_tiles >= 0, "block_sparse_fwd: negative size");
  VEDA_REQUIRE(list_ld >= n_k_tiles, "block_sparse_fwd: list_ld %lld < n_k_tiles %lld",
               (long long)list_ld, (long long)n_k_tiles);
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                   q_stride_s % 8 == 0 && q_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   k_stride_h % 8 == 0 && v_stride_s % 8 == 0 && v_stride_h % 8 == 0 &&
                   o_stride_s % 4 == 0 && o_stride_h % 4 == 0,
               "block_sparse_fwd: rows must be 16-byte aligned");
  const int64_t items = n_heads * n_q_tiles;
  if (items == 0) return VEDA_OK;
  VEDA_REQUIRE(n_k_tiles >= 1 && n_k_tiles <= kMaxBlocks,
               "block_sparse_fwd: n_k_tiles %lld outside [1, %d]", (long long)n_k_tiles, kMaxBlocks);
  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.qs = q_stride_s; p.qh = q_stride_h;
  p.ks = k_stride_s; p.kh = k_stride_h;
  p.vs = v_stride_s; p.vh = v_stride_h;
  p.n_heads = n_heads; p.n_q_tiles = n_q_tiles; p.n_k_tiles = n_k_tiles;
  p.full_cnt = full_cnt; p.full_idx = full_idx;
  p.part_cnt = part_cnt; p.part_idx = part_idx;
  p.list_ld = list_ld;
  p.valid_count = valid_count;
  p.used = 0;
  p.kv_rows = n_k_tiles * kTile;
  p.q_rows = n_q_tiles * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = lse; p.lse_sh = lse_stride_h; p.lse_ss = lse_stride_s;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  fwd_kernel<false><<<(unsigned)items, kThreads, 0, s>>>(p);
  return check_launch("veda_block_sparse_fwd");
}

extern "C" int veda_dense_fwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                              const void* k, int64_t k_stride_s, int64_t k_stride_h,
                              const void* v, int64_t v_stride_s, int64_t v_stride_h,
                              int64_t seq_len, int64_t used, int64_t n_heads, int64_t head_dim,
                              float scale, void* out, int64_t o_stride_s, int64_t o_stride_h,
                              float* lse, int64_t lse_stride_s, int64_t lse_stride_h,
                              void* stream) {
  VEDA_REQUIRE(head_dim == kD, "dense_fwd: head_dim must be 128, got %lld", (long long)head_dim);
  VEDA_REQUIRE(0 <= used && used <= seq_len, "dense_fwd: need 0 <= used <= seq_len");
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                   q_stride_s % 8 == 0 && q_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   k_stride_h % 8 == 0 && v_stride_s % 8 == 0 && v_stride_h % 8 == 0 &&
                   o_stride_s % 4 == 0 && o_stride_h % 4 == 0,
               "dense_fwd: rows must be 16-byte aligned");
  const int64_t n_q_tiles = (seq_len + kTile - 1) / kTile;
  const int64_t items = n_heads * n_q_tiles;
  if (items == 0) return VEDA_OK;
  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.qs = q_stride_s; p.qh = q_stride_h;
  p.ks = k_stride_s; p.kh = k_stride_h;
  p.vs = v_stride_s; p.vh = v_stride_h;
  p.n_heads = n_heads; p.n_q_tiles = n_q_tiles;
  p.n_k_tiles = (used + kTile - 1) / kTile;
  p.used = used;
  p.kv_rows = used;
  p.q_rows = seq_len;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = lse; p.lse_sh = lse_stride_h; p.lse_ss = lse_stride_s;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  fwd_kernel<true><<<(unsigned)items, kThreads, 0, s>>>(p);
  return check_launch("veda_dense_fwd");
}
