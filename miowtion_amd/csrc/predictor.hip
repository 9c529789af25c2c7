// Predictor scoring for gfx950: tile embeddings (feats @ P[h] + mean) and
// block logits (q_hat k_hat^T / sqrt(D) + optional terms), fp32 throughout
// as in the reference (miowtion/veda/predictor.py:251-338).
//
// Both are 64x64-output LDS-tiled fp32 GEMMs (256 threads, 4x4 outputs per
// thread, k-chunks of 16). The weights are decoded in the load path: bf16,
// fp32, or fp8 e4m3 with a per-head scale, turned into the resident bf16
// value bf16(e4m3 * scale) of miowtion/veda/bundle.py:280-297 before use.

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
  embed_kernel<<<grid, 256, 0, s>>>(feats, n_tiles, k_dim, w, w_dtype, w_scale, w_heads, heads,
                                    n_out, residual, out);
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
  logits_kernel<<<grid, 256, 0, s>>>(a, b, n_q, n_k, dim, scale, gain, heads, log_count,
                                     accumulate, out);
  return check_launch("veda_predictor_logits");
}
