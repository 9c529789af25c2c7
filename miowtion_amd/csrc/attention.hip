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
// cross-lane swap (lane ^ 32), the rescale of O is a per-lane scalar, and
// P^T feeds the P.V product straight from the accumulator registers:
//   O^T[d, i] += V^T[d, key] P^T[key, i]   (A = V^T from LDS, B = P^T).
// The MFMA contracts over k, so the order of the 16 keys inside one k-step
// is free; V^T is laid out in LDS in exactly the order the accumulator
// registers hold P^T (keys 16s + 4h + {0..3, 8..11} for lane half h), which
// makes every LDS operand read a single conflict-free 16-byte ds_read.
//
// K / V tiles of the next block are loaded into registers while the current
// block is computed, then written to the other LDS stage (K with a 16-byte
// XOR swizzle, V transposed in registers with byte permutes). One barrier
// per block.

#include "veda_common.h"

namespace veda {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 512;
constexpr int kStageBytes = 2 * kTile * kD * 2;  // K + V^T, 64 KB
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

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
  int64_t kv_rows;   // rows of k / v that may be read
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

// One K or V^T tile of block `j` into staging registers. Threads 0-255 load
// K (8 chunks of 16 bytes each), threads 256-511 load the 8 key rows that
// become one 8x8 transposed block of V^T.
__device__ __forceinline__ void load_stage(const FwdParams& p, int64_t head, int64_t j, int tid,
                                           u32x4 (&st)[8]) {
  const int64_t row0 = j * kTile;
  if (tid < 256) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 4, ch = c & 15;
      const int64_t g = row0 + row;
      st[u] = (g >= 0 && g < p.kv_rows) ? ld16(p.k + g * p.ks + head * p.kh + ch * 8)
                                        : u32x4{0, 0, 0, 0};
    }
  } else {
    const int t = tid - 256;
    const int sh = t >> 4, dg = t & 15;
    const int s = sh >> 1, hh = sh & 1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = 16 * s + 4 * hh + e + (e >= 4 ? 4 : 0);
      const int64_t g = row0 + key;
      st[e] = (g >= 0 && g < p.kv_rows) ? ld16(p.v + g * p.vs + head * p.vh + dg * 8)
                                        : u32x4{0, 0, 0, 0};
    }
  }
}

__device__ __forceinline__ void store_stage(uint8_t* stage, int tid, const u32x4 (&st)[8]) {
  if (tid < 256) {
    uint8_t* kb = stage;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 4, ch = c & 15;
      *reinterpret_cast<u32x4*>(kb + row * 256 + ((ch ^ (row & 15)) << 4)) = st[u];
    }
  } else {
    uint8_t* vb = stage + kTile * kD * 2;
    const int t = tid - 256;
    const int sh = t >> 4, dg = t & 15;
    // out[d] holds the 8 keys (e order) of head-dim 8*dg + d.
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      u32x4 o;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t a = st[2 * m][d >> 1], b = st[2 * m + 1][d >> 1];
        o[m] = (d & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
      }
      *reinterpret_cast<u32x4*>(vb + ((sh * kD) + 8 * dg + d) * 16) = o;
    }
  }
}

template <bool DENSE>
__global__ void __launch_bounds__(kThreads) fwd_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStageBytes];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int qg = wave & 3, kh = wave >> 2;
  const int li = lane & 31, hi = lane >> 5;
  const int64_t item = blockIdx.x;
  const int64_t head = item / p.n_q_tiles;
  const int64_t r = item % p.n_q_tiles;
  const int64_t qrow = r * kTile + 32 * qg + li;

  int nf, nb;
  const int32_t* fl = nullptr;
  const int32_t* pl = nullptr;
  if (DENSE) {
    nf = 0;
    nb = (int)((p.used + kTile - 1) / kTile);
  } else {
    const int64_t li_ = head * p.n_q_tiles + r;
    const int ld = (int)p.list_ld;
    nf = min(max(p.full_cnt[li_], 0), ld);
    nb = nf + min(max(p.part_cnt[li_], 0), ld);
    fl = p.full_idx + li_ * p.list_ld;
    pl = p.part_idx + li_ * p.list_ld;
  }

  // Q^T fragments: lane (li, hi) holds q[qrow, 16 s + 8 hi + 0..7].
  bf16x8 qf[8];
  const bool q_ok = DENSE ? (qrow < p.used) : true;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    u32x4 v = q_ok ? ld16(p.q + qrow * p.qs + head * p.qh + 16 * s + 8 * hi) : u32x4{0, 0, 0, 0};
    qf[s] = as_bf16x8(v);
  }

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  u32x4 st[8];
  auto block_of = [&](int t) -> int64_t {
    if (DENSE) return t;
    return t < nf ? fl[t] : pl[t - nf];
  };
  if (nb > 0) {
    load_stage(p, head, block_of(0), tid, st);
    store_stage(smem, tid, st);
    __syncthreads();
  }
  for (int t = 0; t < nb; ++t) {
    const int64_t j = block_of(t);
    if (t + 1 < nb) load_stage(p, head, block_of(t + 1), tid, st);
    const uint8_t* kb = smem + (t & 1) * kStageBytes;
    const uint8_t* vb = kb + kTile * kD * 2;
    int vc = kTile;
    if (DENSE) {
      const int64_t rem = p.used - j * kTile;
      vc = rem < kTile ? (int)rem : kTile;
    } else if (j < 0 || j >= p.n_k_tiles) {
      vc = 0;  // not a key tile of this layout: contributes nothing
    } else if (t >= nf) {
      vc = p.valid_count[j];
    }

    // S^T for the wave's 64 keys: two 32-key sub-tiles.
    f32x16 sacc[2];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[t2][e] = 0.f;
      const int krow = 64 * kh + 32 * t2 + li;
      const uint8_t* kr = kb + krow * 256;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int ch = 2 * s + hi;
        bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4*>(kr + ((ch ^ (krow & 15)) << 4)));
        sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], sacc[t2], 0, 0, 0);
      }
    }
    // Online softmax in the log2 domain. Register e of sub-tile t2 is key
    // 64 kh + 32 t2 + 8 (e / 4) + 4 hi + e % 4 of this block.
    float mloc = -INFINITY;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = sacc[t2][e] * p.scale_log2;
        if (vc < kTile) {
          const int key = 64 * kh + 32 * t2 + 8 * (e >> 2) + 4 * hi + (e & 3);
          if (key >= vc) x = -INFINITY;
        }
        sacc[t2][e] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float lsum = 0.f;
    u32x4 pk[2][2];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float a = __builtin_amdgcn_exp2f(sacc[t2][8 * kk + 2 * m] - m_use);
          const float b = __builtin_amdgcn_exp2f(sacc[t2][8 * kk + 2 * m + 1] - m_use);
          lsum += a + b;
          pk[t2][kk][m] = pack_bf16x2(a, b);
        }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
    // O^T += V^T P^T over the wave's 4 key-steps of 16 keys.
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int s = 4 * kh + 2 * t2 + kk;  // 16-key group of the block
        const bf16x8 b = as_bf16x8(pk[t2][kk]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const u32x4 av = *reinterpret_cast<const u32x4*>(
              vb + (((2 * s + hi) * kD) + 32 * dt + li) * 16);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), b, o[dt], 0, 0, 0);
        }
      }
    if (t + 1 < nb) store_stage(smem + ((t + 1) & 1) * kStageBytes, tid, st);
    __syncthreads();
  }

  // Merge the two key halves: kh = 1 hands (m, l, O) to kh = 0 through LDS.
  l_run += __shfl_xor(l_run, 32, 64);
  float* red = reinterpret_cast<float*>(smem);  // [qg][64 regs][64 lanes]
  float* ml = red + 4 * 64 * 64;                // [qg][2][32]
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[(qg * 64 + dt * 16 + e) * 64 + lane] = o[dt][e];
    if (hi == 0) {
      ml[qg * 64 + li] = m_run;
      ml[qg * 64 + 32 + li] = l_run;
    }
  }
  __syncthreads();
  if (kh == 1) return;
  const float m1 = ml[qg * 64 + li], l1 = ml[qg * 64 + 32 + li];
  const float m = fmaxf(m_run, m1);
  const float mu = m == -INFINITY ? 0.f : m;
  const float a0 = __builtin_amdgcn_exp2f(m_run - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
  const float l = l_run * a0 + l1 * a1;
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
        v4[rr] = (o[dt][e] * a0 + o1 * a1) * inv;
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

}  // namespace
}  // namespace veda

using namespace veda;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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
  p.n_heads = n_heads; p.n_q_tiles = n_q_tiles; p.n_k_tiles = n_q_tiles;
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
