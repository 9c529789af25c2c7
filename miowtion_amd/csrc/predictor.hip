// Predictor scoring for gfx950: tile embeddings (feats @ P[h] + mean) and
// block logits (q_hat k_hat^T / sqrt(D) + optional terms), fp32 throughout
// as in the reference (miowtion/veda/predictor.py:251-338).
//
// Both run on the matrix cores in fp32 (v_mfma_f32_32x32x2_f32: exact
// products, fp32 sums, as a fp32 GEMM): 64x64 outputs per workgroup, 32x32
// per wave, operands staged through LDS k-contiguous. The MFMA sums over
// its two k in any order, so lane half g supplies k = k0 + 4 g + j to
// product j of a chunk of eight, and each lane reads its four k of A and
// of B as one 16-byte LDS read. The
// weights are decoded in the load path: bf16, fp32, or fp8 e4m3 with a
// per-head scale, turned into the resident bf16 value bf16(e4m3 * scale) of
// miowtion/veda/bundle.py:280-297 before use. Shapes whose k is not a
// multiple of 4, or rows that are not 16-byte aligned, take the
// LDS-tiled VALU form (64x64 outputs, 4x4 per thread, k-chunks of 16).

#include "veda_common.h"

namespace veda {
namespace {

constexpr int kBM = 64, kBN = 64, kBK = 16;

// OCP fp8 e4m3 (the "fn" variant: no infinities, S.1111.111 is NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t s = (b >> 7) & 1u, e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;  // m / 8 * 2^-6
  else if (e == 15 && m == 7) v = __uint_as_float(0x7fc00000u);
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

__device__ __forceinline__ float load_w(const void* w, int dtype, int64_t i, float scale) {
  if (dtype == 0) return bf16_to_f32(static_cast<const uint16_t*>(w)[i]);
  if (dtype == 1) return static_cast<const float*>(w)[i];
  const float v = e4m3_to_f32(static_cast<const uint8_t*>(w)[i]) * scale;
  return bf16_to_f32(f32_to_bf16(v));
}

__global__ void __launch_bounds__(256) embed_kernel(
    const float* __restrict__ feats, int64_t n_tiles, int64_t k_dim, const void* __restrict__ w,
    int w_dtype, const float* __restrict__ w_scale, int64_t w_heads,
    const int64_t* __restrict__ heads, int64_t n_out, int residual, float* __restrict__ out) {
  __shared__ float As[kBK][kBM + 4];
  __shared__ float Bs[kBK][kBN];
  const int64_t hp = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * kBM, n0 = (int64_t)blockIdx.x * kBN;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  int64_t head = heads[hp];
  const bool head_ok = head >= 0 && head < w_heads;
  if (!head_ok) head = 0;
  const float scale = (w_dtype == 2 && head_ok) ? w_scale[head] : 1.f;
  const float* A = feats + hp * n_tiles * k_dim;
  const int64_t wbase = head * k_dim * n_out;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < k_dim; k0 += kBK) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = tid + 256 * u;
      const int am = idx / kBK, ak = idx % kBK;  // A tile 64 x 16
      const int64_t gm = m0 + am, gk = k0 + ak;
      As[ak][am] = (gm < n_tiles && gk < k_dim) ? A[gm * k_dim + gk] : 0.f;
      const int bk = idx / kBN, bn = idx % kBN;  // B tile 16 x 64
      const int64_t gk2 = k0 + bk, gn = n0 + bn;
      Bs[bk][bn] = (gk2 < k_dim && gn < n_out && head_ok)
                       ? load_w(w, w_dtype, wbase + gk2 * n_out + gn, scale) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gm = m0 + ty * 4 + i;
    if (gm >= n_tiles) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + tx * 4 + j;
      if (gn >= n_out) continue;
      float v = acc[i][j];
      if (residual) v += A[gm * k_dim + gn];
      out[(hp * n_tiles + gm) * n_out + gn] = v;
    }
  }
}

__global__ void __launch_bounds__(256) logits_kernel(
    const float* __restrict__ a, const float* __restrict__ b, int64_t n_q, int64_t n_k,
    int64_t dim, float scale, const float* __restrict__ gain, const int64_t* __restrict__ heads,
    const float* __restrict__ log_count, int accumulate, float* __restrict__ out) {
  __shared__ float As[kBK][kBM + 4];
  __shared__ float Bs[kBK][kBN + 4];
  const int64_t hp = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * kBM, n0 = (int64_t)blockIdx.x * kBN;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const float* A = a + hp * n_q * dim;
  const float* B = b + hp * n_k * dim;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < dim; k0 += kBK) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = tid + 256 * u;
      const int rm = idx / kBK, rk = idx % kBK;
      const int64_t gk = k0 + rk;
      const int64_t gm = m0 + rm, gn = n0 + rm;
      As[rk][rm] = (gm < n_q && gk < dim) ? A[gm * dim + gk] : 0.f;
      Bs[rk][rm] = (gn < n_k && gk < dim) ? B[gn * dim + gk] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      float x[4], y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(x[i], y[j], acc[i][j]);
    }
    __syncthreads();
  }
  float g = 0.f;
  if (gain != nullptr) g = gain[heads[hp]];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gm = m0 + ty * 4 + i;
    if (gm >= n_q) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + tx * 4 + j;
      if (gn >= n_k) continue;
      const int64_t o = (hp * n_q + gm) * n_k + gn;
      float v = acc[i][j] * scale;
      if (gain != nullptr) v += g * log_count[gn];
      if (accumulate) v = out[o] + v;
      out[o] = v;
    }
  }
}

// C[h][m][n] = sum_k A[h][m][k] B[h][k][n] on the matrix cores.
// EMBED: A = feats [H'][M][K], B = the head's projection [K][N] (decoded),
// plus the residual A[m][n] when asked; otherwise (logits) B[k][n] =
// b[h][n][k] (k_hat, k-contiguous), then scale, the count term and the
// accumulation into out.
struct PGemm {
  const float* a;
  const float* b;      // logits: k_hat
  const void* w;       // embed: projections
  int w_dtype;
  const float* w_scale;
  int64_t w_heads;
  const int64_t* heads;
  int64_t m, n, k;
  int residual;
  float scale;
  const float* gain;
  const float* log_count;
  int accumulate;
  float* out;
};

constexpr int kKB = 32;       // k per staged block
constexpr int kRow = kKB + 4; // LDS row pitch (floats)

// Workgroup: 64 x 64 outputs, 4 waves of 32 x 32. Per block of 32 k, A's 64
// rows and B's 64 columns go to LDS k-contiguous ([row][k], B transposed:
// [n][k]) with coalesced 16-byte loads (the projection is decoded on the
// way); the next block's loads are in flight while the current block's 16
// products per wave run from LDS. Rows and columns past the matrix are
// staged from clamped real rows and not stored.
template <bool EMBED>
__global__ void __launch_bounds__(256) pgemm_kernel(PGemm p) {
  __shared__ __attribute__((aligned(16))) float As[2][kBM][kRow];
  __shared__ __attribute__((aligned(16))) float Bs[2][kBN][kRow];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 31, g = lane >> 5;
  const int64_t hp = blockIdx.z;
  const int64_t mb = (int64_t)blockIdx.y * kBM, nb = (int64_t)blockIdx.x * kBN;
  const int wm = 32 * (wave >> 1), wn = 32 * (wave & 1);
  int64_t head = 0;
  bool head_ok = true;
  float wscale = 1.f;
  if (EMBED) {
    head = p.heads[hp];
    head_ok = head >= 0 && head < p.w_heads;
    if (!head_ok) head = 0;
    wscale = (p.w_dtype == 2 && head_ok) ? p.w_scale[head] : 1.f;
  }
  const int64_t wbase = head * p.k * p.n;
  // staging: thread t moves k 4 (t % 8) .. + 3 of rows t / 8 and t / 8 + 32
  // of A (and of k_hat); for the projection, k t / 8 of columns 8 (t % 8) ..
  // + 7
  const int sr = tid >> 3, sk = 4 * (tid & 7);
  struct Stage {
    f32x4 a[2], b[2];
    float w[8];
  };
  auto load = [&](Stage& st, int64_t k0) {
    f32x4 (&ra)[2] = st.a;
    f32x4 (&rb)[2] = st.b;
    float (&rw)[8] = st.w;
    const int64_t kk = k0 + sk;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t gm = min(mb + sr + 32 * h, p.m - 1);
      ra[h] = kk < p.k ? *reinterpret_cast<const f32x4*>(p.a + (hp * p.m + gm) * p.k + kk)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
      if (!EMBED) {
        const int64_t gn = min(nb + sr + 32 * h, p.n - 1);
        rb[h] = kk < p.k ? *reinterpret_cast<const f32x4*>(p.b + (hp * p.n + gn) * p.k + kk)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    if (EMBED) {
      const int64_t wk = k0 + sr;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t gn = nb + 8 * (tid & 7) + j;
        rw[j] = (wk < p.k && gn < p.n && head_ok) ? load_w(p.w, p.w_dtype, wbase + wk * p.n + gn, wscale)
                                                 : 0.f;
      }
    }
  };
  auto store = [&](const Stage& st, int buf) {
    const f32x4 (&ra)[2] = st.a;
    const f32x4 (&rb)[2] = st.b;
    const float (&rw)[8] = st.w;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<f32x4*>(&As[buf][sr + 32 * h][sk]) = ra[h];
      if (!EMBED) *reinterpret_cast<f32x4*>(&Bs[buf][sr + 32 * h][sk]) = rb[h];
    }
    if (EMBED) {
#pragma unroll
      for (int j = 0; j < 8; ++j) Bs[buf][8 * (tid & 7) + j][sr] = rw[j];
    }
  };
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  const int nblk = (int)((p.k + kKB - 1) / kKB);
  auto products = [&](int buf) {
#pragma unroll
    for (int c = 0; c < kKB / 8; ++c) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&As[buf][wm + li][8 * c + 4 * g]);
      const f32x4 b = *reinterpret_cast<const f32x4*>(&Bs[buf][wn + li][8 * c + 4 * g]);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], acc, 0, 0, 0);
    }
  };
  // blocks b + 1 and b + 2 are in registers or in flight while block b is
  // in LDS being multiplied: the loads run two blocks ahead of their use
  Stage r0, r1;
  load(r0, 0);
  store(r0, 0);
  load(r0, kKB);           // block 1 (zeros past k)
  load(r1, 2 * kKB);       // block 2
  __syncthreads();
  for (int kb = 0; kb < nblk; kb += 2) {
    products(0);
    if (kb + 1 >= nblk) break;
    store(r0, 1);          // block kb + 1
    load(r0, (int64_t)(kb + 3) * kKB);
    __syncthreads();
    products(1);
    if (kb + 2 >= nblk) break;
    store(r1, 0);          // block kb + 2
    load(r1, (int64_t)(kb + 4) * kKB);
    __syncthreads();
  }
  // lane (li, g) holds column nb + wn + li, rows mb + wm + 8 (e / 4) + 4 g + e % 4
  const int64_t gn = nb + wn + li;
  if (gn >= p.n) return;
  float gterm = 0.f;
  if (!EMBED && p.gain != nullptr) gterm = p.gain[p.heads[hp]] * p.log_count[gn];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int64_t gm = mb + wm + 8 * (e >> 2) + 4 * g + (e & 3);
    if (gm >= p.m) continue;
    const int64_t o = (hp * p.m + gm) * p.n + gn;
    float v = acc[e];
    if (EMBED) {
      if (p.residual) v += p.a[(hp * p.m + gm) * p.k + gn];
    } else {
      v = v * p.scale;
      if (p.gain != nullptr) v += gterm;
      if (p.accumulate) v = p.out[o] + v;
    }
    p.out[o] = v;
  }
}

}  // namespace
}  // namespace veda

using namespace veda;

extern "C" int veda_predictor_embed(const float* feats, int64_t n_heads, int64_t n_tiles,
                                    int64_t k_dim, const void* w, int w_dtype,
                                    const float* w_scale, int64_t w_heads, const int64_t* heads,
                                    int64_t n_out, int residual, float* out, void* stream) {
  VEDA_REQUIRE(w_dtype >= 0 && w_dtype <= 2, "predictor_embed: unknown weight dtype %d", w_dtype);
  VEDA_REQUIRE(w_dtype != 2 || w_scale != nullptr, "predictor_embed: e4m3 needs a scale");
  VEDA_REQUIRE(!residual || k_dim >= n_out, "predictor_embed: residual needs k_dim >= n_out");
  VEDA_REQUIRE(n_heads >= 0 && n_tiles >= 0 && k_dim >= 1 && n_out >= 1,
               "predictor_embed: bad sizes");
  if (n_heads == 0 || n_tiles == 0) return VEDA_OK;
  dim3 grid((unsigned)((n_out + kBN - 1) / kBN), (unsigned)((n_tiles + kBM - 1) / kBM),
            (unsigned)n_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (k_dim % 4 == 0 && (reinterpret_cast<uintptr_t>(feats) & 15) == 0) {
    PGemm p{};
    p.a = feats; p.w = w; p.w_dtype = w_dtype; p.w_scale = w_scale; p.w_heads = w_heads;
    p.heads = heads; p.m = n_tiles; p.n = n_out; p.k = k_dim; p.residual = residual;
    p.out = out;
    pgemm_kernel<true><<<grid, 256, 0, s>>>(p);
  } else {
    embed_kernel<<<grid, 256, 0, s>>>(feats, n_tiles, k_dim, w, w_dtype, w_scale, w_heads, heads,
                                      n_out, residual, out);
  }
  return check_launch("veda_predictor_embed");
}

extern "C" int veda_predictor_logits(const float* a, const float* b, int64_t n_heads, int64_t n_q,
                                     int64_t n_k, int64_t dim, float scale, const float* gain,
                                     const int64_t* heads, const float* log_count, int accumulate,
                                     float* out, void* stream) {
  VEDA_REQUIRE(gain == nullptr || (heads != nullptr && log_count != nullptr),
               "predictor_logits: gain needs heads and log_count");
  VEDA_REQUIRE(n_heads >= 0 && n_q >= 0 && n_k >= 0 && dim >= 1, "predictor_logits: bad sizes");
  if (n_heads == 0 || n_q == 0 || n_k == 0) return VEDA_OK;
  dim3 grid((unsigned)((n_k + kBN - 1) / kBN), (unsigned)((n_q + kBM - 1) / kBM),
            (unsigned)n_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0) {
    PGemm p{};
    p.a = a; p.b = b; p.heads = heads; p.m = n_q; p.n = n_k; p.k = dim; p.scale = scale;
    p.gain = gain; p.log_count = log_count; p.accumulate = accumulate; p.out = out;
    pgemm_kernel<false><<<grid, 256, 0, s>>>(p);
  } else {
    logits_kernel<<<grid, 256, 0, s>>>(a, b, n_q, n_k, dim, scale, gain, heads, log_count,
                                       accumulate, out);
  }
  return check_launch("veda_predictor_logits");
}
