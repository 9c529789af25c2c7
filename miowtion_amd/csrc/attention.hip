// Flash-attention forwards for gfx950 (head_dim 128, bf16 in, fp32
// accumulate). Two kernels share the step, fragment and load code below:
//   hfwd_kernel  the teacher's pass over all key tiles in tile order with
//                the dense output (and the block heat statistics);
//   tstats_kernel the same pass without the output (LSE and statistics
//                only), four query tiles per K pass;
//   sfwd_kernel  the block-sparse forward, the zero-order compensation and
//                the dense forward of packed rows (two 4-wave workgroups
//                per CU, described at its section).
//
// hfwd_kernel: workgroup = one (head, 128-row query tile), 8 waves, 1 per CU:
//   wave w: query group qg = w & 3 (32 query rows), key half kh = w >> 2;
//   waves w and w + 4 share a SIMD, so one wave's softmax can overlap the
//   other's MFMAs. The two key halves keep separate online-softmax states
//   and are merged through LDS at the end.
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
// K and V go from HBM straight into LDS (global_load_lds_dwordx4: lane l of
// a wave writes bytes [16 l, 16 l + 16) of a 1 KB segment), no register
// staging and no transposing stores. Both keep their natural [key][head_dim]
// row layout with the 16-byte chunks of row r permuted:
//   K: chunk c at position c ^ (r & 15)   -> the 16-byte K fragment reads of
//      32 consecutive rows are conflict-free;
//   V: chunk c at position c ^ 4 (r & 3)  -> the V^T fragments, assembled by
//      two ds_read_b64_tr_b16 (lane i of a 16-lane group receives element
//      (i mod 4) of source lane 4 j + i / 4, j = 0..3), are conflict-free.
// The pipeline over the kept blocks is described at the half-block section.

#include <type_traits>

#include "veda_common.h"
#include "veda_pipeline.h"

namespace veda {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 512;
constexpr int kTileBytes = kTile * kD * 2;       // 32 KB: one K or V tile
constexpr int kMaxBlocks = 2048;                 // key tiles per row (FA4's cap)
// LDS offset in ring slot 1 of the Q fragments a narrow walk hands from wave
// 0 to wave 1 (8 KB, past the set-up's 12 KB step-list scratch)
constexpr int kNarrowQ = 16384;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.f;             // log2 units


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
  int64_t used;      // dense rows: real rows
  int64_t q_rows;    // dense rows: rows of q / out / lse that exist
  float scale_log2;  // softmax scale * log2(e)
  uint16_t* out;
  int64_t os, oh;
  float* lse;
  int64_t lse_sh, lse_ss;
  // All-tiles walk only: query tile of item r (NULL: tile r), and the
  // per-(key tile, query row) block statistic [H'][n_k][items * 128] in
  // log2 units (block log-sum-exp for heat 'sum', block max for 'max').
  const int64_t* q_tiles;
  int64_t q_tiles_held;  // tiles q holds; an item whose q_tiles entry is outside reads zeros
  // Virtual keys (zero-order compensation) only: the kept-block mask
  // [H'][items][n_k] (bytes), the tile summaries kc / vc ([n_k][H'][D],
  // strides cs, ch), and for the compensation of a given output, that
  // output o_kept and its LSE lse_kept.
  const uint8_t* keep;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t cs, ch;
  const uint16_t* o_kept;
  int64_t oks, okh;
  const float* lse_kept;
  int64_t lk_h, lk_s;
  float* part;
  int64_t part_sh, part_st;
  int64_t front;  // sparse walks: query tiles [n_q - front, n_q) of every head go first
  // Sparse walk in sequence order (veda_block_sparse_fwd_seq; NULL: tile
  // order): query slot s reads q row seq_q[s] and writes out row seq_o[s]
  // of head seq_heads[h'], q being [seq_rows, seq_heads_n, D] and out
  // [out_rows, seq_heads_n, D]. A slot whose slot_ok is 0, or whose row or
  // head is out of range, reads zeros and writes nothing (the semantics of
  // the gather and scatter kernels).
  const int64_t* seq_q;
  const int64_t* seq_o;
  const int32_t* slot_ok;
  const int64_t* seq_heads;
  int64_t seq_rows, seq_heads_n, out_rows;
};

// Block statistic collected for the teacher heat: none, log-sum-exp, max.
enum Heat { kNoHeat = 0, kHeatSum = 1, kHeatMax = 2 };
constexpr int32_t kTileEnd = 1 << 30;  // step-list flag: last step of its key tile


// Per-wave state: Q^T fragments of the wave's 32 rows (lane (li, hi) holds
// q[row 32 qg + li, 16 s + 8 hi .. + 7]), the O^T accumulators
// (O^T[d in 32 dt .. + 31][row]) and the online-softmax state of its rows.
struct WaveState {
  bf16x8 qf[8];
  f32x16 o[4];
  float m_run, l_run;
  float mu;     // exponent offset of the last step computed
  float blk;    // heat: the current key tile's partial (sum relative to mu, or max)
};

// ---------------------------------------------------------------------------
// Half-block pipeline.
//
// The unit of the pipeline is a step: 64 keys of one key tile, K and V
// together 32 KB. Four LDS slots form a ring, so three steps are in flight
// while one is computed (96 KB per CU; with a random block list most K/V
// reads miss L2 and come over the fabric, which needs that depth to run at
// its bandwidth).
//
// A step loads and computes only what the key tile holds: rows at or past
// the tile's valid count are padding (masked by definition), so their 1 KB
// segments are not fetched from HBM (the load is redirected to rows already
// being fetched, which keeps every wave's load count fixed for the vmcnt
// waits, and writes copies of real rows into those LDS rows, so every row a
// step reads was written by that step), and the upper half of a tile with
// at most 64 valid keys is no step at all. Rows past the valid count only
// ever meet masked keys (p = 0).
//
// In each step wave (qg, kh) takes keys 32 kh .. 32 kh + 31 of the half:
// S^T = K Q^T (8 MFMAs), one online-softmax step over its 32 keys, and
// O^T += V^T P^T (8 MFMAs); a wave whose 32 keys are all padding skips the
// step. The two key halves merge at the end.

constexpr int kSlotBytes = 2 * kHalfBytes;      // 32 KB: K + V
static_assert(3 * kMaxBlocks * 2 <= kNarrowQ && kNarrowQ + 8 * 64 * 16 <= kSlotBytes,
              "narrow-walk Q fragments overlap the step-list scratch or leave the slot");

// Per-lane byte offsets of the HBM -> LDS loads of one step. Wave w fills K
// and V segments 2w, 2w + 1 (1 KB = rows 4 seg .. 4 seg + 3 of the half);
// lane l loads row 4 seg + l / 16, LDS chunk l % 16, which holds logical
// chunk (l % 16) ^ (row & 15) of K and (l % 16) ^ 4 (row & 3) of V. `skip`
// offsets re-read rows l / 16 instead (for segments wholly past the valid
// count; what they write is never used).
struct HDma {
  uint32_t k[2], v[2], k_skip[2], v_skip[2];
};

__device__ __forceinline__ HDma hdma_offsets(int64_t ks, int64_t vs, int wave, int lane) {
  HDma d;
  const int lr = lane >> 4, pc = lane & 15;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = 4 * (2 * wave + u) + lr;
    const int kc = (pc ^ (row & 15)) << 3, vc = (pc ^ ((row & 3) << 2)) << 3;
    d.k[u] = (uint32_t)((row * ks + kc) * 2);
    d.v[u] = (uint32_t)((row * vs + vc) * 2);
    d.k_skip[u] = (uint32_t)((lr * ks + kc) * 2);
    d.v_skip[u] = (uint32_t)((lr * vs + vc) * 2);
  }
  return d;
}


// Issues the loads of the step at key row row0 (64 rows, the first vch of
// them valid) into `slot`.
__device__ __forceinline__ void issue_step(const uint16_t* kbase, const uint16_t* vbase,
                                           const FwdParams& p, const HDma& d, int64_t row0,
                                           int vch, int wave, int lane, lds_u8* slot) {
  const char* kb = reinterpret_cast<const char*>(kbase + row0 * p.ks);
  const char* vb = reinterpret_cast<const char*>(vbase + row0 * p.vs);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int seg = 2 * wave + u;
    const bool live = 4 * seg < vch;
    dma16(kb, live ? d.k[u] : d.k_skip[u], slot + seg * 1024);
    dma16(vb, live ? d.v[u] : d.v_skip[u], slot + kHalfBytes + seg * 1024);
  }
}

// Per-lane LDS offsets of the fragment reads inside a slot.
struct HFrag {
  uint32_t k[8];  // K row 32 kh + li, logical chunk 2k + hi
  uint32_t v[4];  // V^T fragment base per dt (V region included)
};

__device__ __forceinline__ HFrag hfrag_offsets(int kh, int lane) {
  HFrag f;
  const int li = lane & 31, hi = lane >> 5;
  const uint32_t krow = (32 * kh + li) * 256, x = (hi ^ (li & 15)) << 4;
#pragma unroll
  for (int k = 0; k < 8; ++k) f.k[k] = krow + (x ^ (k << 5));
  // V^T of lane (16-lane group g = (hi, dh), i): transposed reads of rows
  // 16 sg + 4 hi + i / 4 (+ 8), head-dims 32 dt + 16 dh + 4 (i % 4) .. + 3,
  // sg = 2 kh + kk the 16-key group.
  const int i16 = lane & 15, q4 = i16 >> 2, dh = (lane >> 4) & 1;
  const uint32_t vb =
      (4 * hi + q4) * 256 + (((2 * dh + ((i16 >> 1) & 1)) << 4) | (q4 << 6)) + (i16 & 1) * 8;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) f.v[dt] = kHalfBytes + 2 * kh * 16 * 256 + (vb ^ (dt << 6));
  return f;
}

// One step for this wave's 32 rows and 32 keys from `slot`; keys at or past
// vch (of the half) are masked.
template <int HEAT>
__device__ __forceinline__ void hstep(const lds_u8* slot, const HFrag& f, float c, int vch,
                                      int kh, int hi, WaveState& w) {
  u32x4 kf[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    kf[k] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(slot + f.k[k]);
  f32x16 s;
#pragma unroll
  for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[k]), w.qf[k], s, 0, 0, 0);
  // Register e holds key 32 kh + 8 (e / 4) + 4 hi + e % 4 of the half.
  if (vch < 32 * (kh + 1)) {
    const int lim = vch - 32 * kh - 4 * hi;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (8 * (e >> 2) + (e & 3) >= lim) s[e] = -INFINITY;
  }
  // Online softmax step in the log2 domain: p = exp2(s * c - m). The
  // reference max m rises only when the step's row max passes it by more
  // than kRescaleSlack (p then stays <= 2^kRescaleSlack, exact in fp32 and
  // bf16), so the O rescale is skipped for most steps; numerator and
  // denominator share m.
  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, s[e]);
  const float mraw = half_swap_max(mloc);  // unscaled row max over the wave's 32 keys
  mloc = mraw * c;
  const float m_new = mloc > w.m_run + kRescaleSlack ? mloc : w.m_run;
  const float mu = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(w.m_run - mu);
  w.m_run = m_new;
  w.mu = mu;
  // heat 'max': the wave's unscaled row max over its keys of the tile
  if (HEAT == kHeatMax) w.blk = fmaxf(w.blk, mraw);
  float ps[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) ps[e] = __builtin_amdgcn_exp2f(fmaf(s[e], c, -mu));
  float l4[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) l4[g] = (ps[4 * g] + ps[4 * g + 1]) + (ps[4 * g + 2] + ps[4 * g + 3]);
  const float lsum = (l4[0] + l4[1]) + (l4[2] + l4[3]);
  w.l_run = fmaf(w.l_run, alpha, lsum);
  // heat 'sum': this lane's 16 keys, relative to mu like l
  if (HEAT == kHeatSum) w.blk = fmaf(w.blk, alpha, lsum);
  u32x4 pk[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int m = 0; m < 4; ++m) pk[kk][m] = pack_bf16x2(ps[8 * kk + 2 * m], ps[8 * kk + 2 * m + 1]);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) w.o[dt][e] *= alpha;
  }
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const lds_u8* vs = slot + kk * 16 * 256;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vs + f.v[dt]));
      const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vs + 8 * 256 + f.v[dt]));
      const bf16x8 a =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7));
      w.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_bf16x8(pk[kk]), w.o[dt], 0, 0, 0);
    }
  }
}


// The teacher's pass: every key tile of a tile layout in order, its padding
// rows masked, with the block statistic of the heat and the dense output.
template <int HEAT>
__global__ void __launch_bounds__(kThreads) hfwd_kernel(FwdParams p) {
  // The steps are 16-bit (tile, half) entries plus a byte per tile of
  // valid counts.
  constexpr int kSlot = kSlotBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t slot0[kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t slot1[kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t slot2[kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t slot3[kSlot];
  __shared__ uint16_t tile_steps[2 * kMaxBlocks];  // (key tile << 1) | half
  __shared__ uint8_t tile_valid[kMaxBlocks];
  __shared__ int32_t step_total;
  __shared__ float lbuf[2][4][32];  // heat: kh = 1 hands its key-tile partials to kh = 0
  lds_u8* sl0 = (lds_u8*)slot0;
  lds_u8* sl1 = (lds_u8*)slot1;
  lds_u8* sl2 = (lds_u8*)slot2;
  lds_u8* sl3 = (lds_u8*)slot3;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int qg = wave & 3, kh = wave >> 2;
  const int li = lane & 31, hi = lane >> 5;
  const int64_t item = blockIdx.x;
  const int64_t head = item / p.n_q_tiles;
  const int64_t r = item % p.n_q_tiles;
  const int64_t qrow = r * kTile + 32 * qg + li;  // row of out / lse / part
  // row of q: item r reads query tile q_tiles[r]
  const int64_t qtile = p.q_tiles != nullptr ? p.q_tiles[r] : r;
  const bool qtile_ok = qtile >= 0 && qtile < p.q_tiles_held;
  const int64_t qsrc = (qtile_ok ? qtile : 0) * kTile + 32 * qg + li;

  // The ring needs no clearing: every step's loads write all 64 rows of
  // its slot (segments past the valid count re-read real rows), so an MFMA
  // only ever reads rows its own step wrote.

  // Steps: every key tile in order, its steps consecutive: the first half,
  // then the second half when more than 64 keys are valid; the tile's last
  // step carries kTileEnd. An empty tile is one step with no valid key.
  {
    if (wave == 0) {
      const int nk = (int)p.n_k_tiles;
      int base = 0;
      for (int j0 = 0; j0 < nk; j0 += 64) {
        const int j = j0 + lane;
        const int vc = j < nk ? min(max(p.valid_count[j], 0), kTile) : 0;
        const bool two = j < nk && vc > kHalf;
        const uint64_t bal = __ballot(two);
        const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
        if (j < nk) {
          const int at = base + lane + rank;
          tile_valid[j] = (uint8_t)vc;
          tile_steps[at] = (uint16_t)(j << 1);
          if (two) tile_steps[at + 1] = (uint16_t)((j << 1) | 1);
        }
        base += min(64, nk - j0) + __builtin_popcountll(bal);
      }
      if (lane == 0) step_total = base;
    }
  }

  WaveState w;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    u32x4 v = qtile_ok ? ld16(p.q + qsrc * p.qs + head * p.qh + 16 * s + 8 * hi) : u32x4{0, 0, 0, 0};
    w.qf[s] = as_bf16x8(v);
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" : : "v"(w.qf[s]));
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) w.o[dt][e] = 0.f;
  w.m_run = -INFINITY;
  w.l_run = 0.f;
  w.mu = 0.f;
  w.blk = HEAT == kHeatMax ? -INFINITY : 0.f;
  __syncthreads();  // step list and step count ready
  const int n_steps = __builtin_amdgcn_readfirstlane(step_total);

  // Step word of step u: (first key row << 7) | valid keys | kTileEnd.
  auto step_word = [&](int u) -> int32_t {
    const int e = __builtin_amdgcn_readfirstlane(tile_steps[u]);
    const int j = e >> 1, half = e & 1;
    const int vc = __builtin_amdgcn_readfirstlane(tile_valid[j]);
    const int vch = half ? vc - kHalf : min(vc, kHalf);
    return ((j * kTile + half * kHalf) << 7) | vch | ((half || vc <= kHalf) ? kTileEnd : 0);
  };
  // (first key row, valid keys) of step u
  auto step_row = [&](int u) -> int64_t { return (int64_t)((step_word(u) >> 7) & 0x7FFFFF); };
  auto step_vch = [&](int u) -> int { return step_word(u) & 127; };
  const uint16_t* kbase = p.k + head * p.kh;
  const uint16_t* vbase = p.v + head * p.vh;
  const float c = p.scale_log2;
  const HDma dma = hdma_offsets(p.ks, p.vs, wave, lane);
  const HFrag frag = hfrag_offsets(kh, lane);

  // a step with no valid key (an empty tile) loads the tile's first rows,
  // which exist; its keys are all masked
  auto load_step = [&](int u, lds_u8* slot) {
    issue_step(kbase, vbase, p, dma, step_row(u), step_vch(u), wave, lane, slot);
  };
  // Prologue: steps 0, 1, 2 into slots 0, 1, 2.
  if (n_steps > 0) load_step(0, sl0);
  if (n_steps > 1) load_step(1, sl1);
  if (n_steps > 2) load_step(2, sl2);
  // Step u: wait for its own loads (every step is 4 loads per wave; the
  // loads of steps u+1, u+2 may stay in flight), barrier, refill the slot
  // step u-1 used with step u+3, compute step u.
  // The barrier is a bare s_barrier: __syncthreads() would also fence
  // memory, i.e. wait for every load in flight. LDS is coherent inside the
  // workgroup, the step's DMA is complete in every wave once each has waited
  // for its own loads, and every fragment read of the previous step has been
  // consumed by an MFMA before its wave reaches the barrier.
  auto wait_step = [&](int u) {
    // loads per wave per step: 4 (K and V)
    if (u + 2 < n_steps) VEDA_WAIT_VM(8);
    else if (u + 1 < n_steps) VEDA_WAIT_VM(4);
    else VEDA_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
  };
  // A wave whose 32 keys of the step are all padding skips the step: all
  // its scores would be -inf, which leaves m, l and O unchanged.
  // Heat partials. At the end of a key tile each wave turns its partial
  // into a log2 statistic of its rows over its keys of the tile: the
  // log-sum-exp ('sum': log2 of the sum, relative to mu, plus mu) or the
  // max ('max'). kh = 1 leaves it in LDS; kh = 0 combines it with its own
  // after the next barrier and writes one value per (key tile, row).
  int pend_j = -1;
  float pend_l = 0.f;
  auto flush_tile = [&](int j) {
    float l;
    if (HEAT == kHeatSum) {
      const float tot = half_swap_sum(w.blk);
      l = tot > 0.f ? __log2f(tot) + w.mu : -INFINITY;
      w.blk = 0.f;
    } else {
      // the reference rounds the unscaled max to the input dtype (bf16) and
      // scales after it (block_heat_triton.py:131-133, heatmap.py:88-95)
      l = bf16_to_f32(f32_to_bf16(w.blk)) * c;
      w.blk = -INFINITY;
    }
    if (kh == 1) {
      if (hi == 0) lbuf[j & 1][qg][li] = l;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // visible at the next barrier
    } else {
      pend_l = l;
      pend_j = j;
    }
  };
  auto write_pending = [&]() {
    const float l1 = lbuf[pend_j & 1][qg][li];
    float l;
    if (HEAT == kHeatSum) {
      const float a = fmaxf(pend_l, l1), b = fminf(pend_l, l1);
      l = a == -INFINITY ? -INFINITY : a + __log2f(1.f + __builtin_amdgcn_exp2f(b - a));
    } else {
      l = fmaxf(pend_l, l1);
    }
    if (hi == 0) p.part[head * p.part_sh + (int64_t)pend_j * p.part_st + qrow] = l;
    pend_j = -1;
  };
  auto compute_step = [&](int u, const lds_u8* slot) {
    const int vch = step_vch(u);
    if (HEAT != kNoHeat && kh == 0 && pend_j >= 0) write_pending();
    if (vch > 32 * kh) hstep<HEAT>(slot, frag, c, vch, kh, hi, w);
    if (HEAT != kNoHeat) {
      const int32_t word = step_word(u);
      if (word & kTileEnd) flush_tile((word >> 7 & 0x7FFFFF) / kTile);
    }
  };
  for (int u = 0; u < n_steps; u += 4) {
    wait_step(u);
    if (u + 3 < n_steps) load_step(u + 3, sl3);
    compute_step(u, sl0);
    if (u + 1 >= n_steps) break;
    wait_step(u + 1);
    if (u + 4 < n_steps) load_step(u + 4, sl0);
    compute_step(u + 1, sl1);
    if (u + 2 >= n_steps) break;
    wait_step(u + 2);
    if (u + 5 < n_steps) load_step(u + 5, sl1);
    compute_step(u + 2, sl2);
    if (u + 3 >= n_steps) break;
    wait_step(u + 3);
    if (u + 6 < n_steps) load_step(u + 6, sl2);
    compute_step(u + 3, sl3);
  }
  __syncthreads();  // every wave is done reading the ring
  if (HEAT != kNoHeat && kh == 0 && pend_j >= 0) write_pending();

  // Merge the two key halves: kh = 1 hands (m, l, O) to kh = 0 through LDS.
  w.l_run = half_swap_sum(w.l_run);
  // [qg & 1][64 regs][64 lanes] in slot 0 (qg < 2) or slot 1 (qg >= 2)
  float* red = reinterpret_cast<float*>(qg < 2 ? slot0 : slot1) + (qg & 1) * 64 * 64;
  float* ml = reinterpret_cast<float*>(slot2);  // [qg][m | l][32]
  if (kh == 1) {
    {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[(dt * 16 + e) * 64 + lane] = w.o[dt][e];
    }
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
  const float a0 = __builtin_amdgcn_exp2f(w.m_run - mu);
  const float a1 = __builtin_amdgcn_exp2f(m1 - mu);
  const float l = w.l_run * a0 + l1 * a1;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = p.out + qrow * p.os + head * p.oh;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v4[4];
      const int d = 32 * dt + 8 * g + 4 * hi;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int e = 4 * g + rr;
        const float o1 = red[(dt * 16 + e) * 64 + lane];
        v4[rr] = (w.o[dt][e] * a0 + o1 * a1) * inv;
      }
      uint32_t w0 = pack_bf16x2(v4[0], v4[1]), w1 = pack_bf16x2(v4[2], v4[3]);
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2*>(orow + d) = u32x2{w0, w1};
    }
  if (p.lse != nullptr && hi == 0) {
    const float lse = l > 0.f ? (m + __log2f(l)) * kLn2 : -INFINITY;
    p.lse[head * p.lse_sh + qrow * p.lse_ss] = lse;
  }
}

// ---------------------------------------------------------------------------
// Sparse forward, two workgroups per CU.
//
// Workgroup = one (head, query tile), 4 waves; wave w owns query rows
// 32 w .. 32 w + 31 and all 64 keys of every step (two 32-key sub-blocks,
// A = keys 0..31, B = keys 32..63 of the step), so a wave's rows are
// complete at the end and no key halves are merged. The ring is two K + V
// slots (64 KB) with one step in flight, the step list 16-bit (key tile,
// half, full-list flag) entries with a byte table of valid counts: 74 KB of
// LDS, so two workgroups share a CU. Their waves are not tied by a barrier,
// so the two waves of a SIMD drift apart and fill each other's stalls.

constexpr int kThreads2 = 256;
constexpr uint16_t kVoidStep = 0xFFFF;  // list entry outside [0, n_k): no valid key
constexpr uint16_t kPairStep = 0x8000;  // step entry flag: a pair of ragged halves
// Workgroups of the sparse walk resident at once on MI355X (256 CUs, two
// each): the period of the walks' rotation over the key tiles.
constexpr int kSweepWorkgroups = 512;

// Per-lane byte offsets of this wave's eight 1 KB segments of a step
// (segments 4 w + u, u = 0..3, of K and of V: rows 4 seg + l / 16), and of
// their redirect (rows l / 16) for segments wholly past the valid count.
struct SDma {
  uint32_t k[4], v[4], k_skip[4], v_skip[4];
};

// Source offsets of wave `wave`'s four 1 KB segments (rows 16 wave .. + 15
// of the 64-row slot). Waves 0, 1 fill sub-block a (slot rows 0 .. 31),
// waves 2, 3 sub-block b (slot rows 32 .. 63); each pair's offsets count
// from its own sub-block's first source row, so the two sub-blocks of a
// step may come from different key tiles.
__device__ __forceinline__ SDma sdma_offsets(int64_t ks, int64_t vs, int wave, int lane) {
  SDma d;
  const int lr = lane >> 4, pc = lane & 15;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = 4 * (4 * wave + u) + lr;
    const int src = row - (wave >= 2 ? 32 : 0);
    const int kc = (pc ^ (row & 15)) << 3, vc = (pc ^ ((row & 3) << 2)) << 3;
    d.k[u] = (uint32_t)((src * ks + kc) * 2);
    d.v[u] = (uint32_t)((src * vs + vc) * 2);
    d.k_skip[u] = (uint32_t)((lr * ks + kc) * 2);
    d.v_skip[u] = (uint32_t)((lr * vs + vc) * 2);
  }
  return d;
}

// Scores of a 32-key sub-block past its first `lim` keys set to -inf (lim >=
// 32: none; lim <= 0: all); register e holds key 8 (e / 4) + 4 hi + e % 4.
__device__ __forceinline__ void mask_scores(f32x16& s, int lim, int hi) {
  if (lim < 32) {
    const int l = lim - 4 * hi;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (8 * (e >> 2) + (e & 3) >= l) s[e] = -INFINITY;
  }
}

// Scores of one 32-key sub-block, masked past `lim` keys of it.
__device__ __forceinline__ f32x16 sub_scores(const lds_u8* slot, const HFrag& f,
                                             const WaveState& w, int lim, int hi) {
  u32x4 kf[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    kf[k] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(slot + f.k[k]);
  f32x16 s;
#pragma unroll
  for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[k]), w.qf[k], s, 0, 0, 0);
  mask_scores(s, lim, hi);
  return s;
}

// Scores of both 32-key sub-blocks of a step, as two interleaved MFMA
// chains (each fragment read has the other chain's product to hide behind),
// then the masks of sub-blocks with fewer than 32 valid keys.
__device__ __forceinline__ void pair_scores(const lds_u8* slot, const HFrag& fa, const HFrag& fb,
                                            const WaveState& w, int la, int lb, int hi,
                                            f32x16& sa, f32x16& sb) {
#pragma unroll
  for (int e = 0; e < 16; ++e) sa[e] = sb[e] = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const u32x4 ka = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(slot + fa.k[k]);
    const u32x4 kb = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(slot + fb.k[k]);
    sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka), w.qf[k], sa, 0, 0, 0);
    sb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kb), w.qf[k], sb, 0, 0, 0);
  }
  // issue order: the reads of k + 2 before the products of k (more reads
  // ahead than the compiler's own schedule keeps; all 16 ahead was slower)
  __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  mask_scores(sa, la, hi);
  mask_scores(sb, lb, hi);
}

// The same products with hook(k) between them: the fragment reads of
// product k + 2 are placed before product k and hook(k) before the reads of
// k + 2, in program order (a hook that branches ends the scheduling region,
// so the order is written out instead of left to scheduling hints).
template <typename Hook>
__device__ __forceinline__ void pair_scores_hooked(const lds_u8* slot, const HFrag& fa,
                                                   const HFrag& fb, const WaveState& w, int la,
                                                   int lb, int hi, f32x16& sa, f32x16& sb,
                                                   Hook hook) {
  typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
#pragma unroll
  for (int e = 0; e < 16; ++e) sa[e] = sb[e] = 0.f;
  u32x4 ka[8], kb[8];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    ka[k] = *reinterpret_cast<lds_u32x4>(slot + fa.k[k]);
    kb[k] = *reinterpret_cast<lds_u32x4>(slot + fb.k[k]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    hook(k);
    if (k + 2 < 8) {
      ka[k + 2] = *reinterpret_cast<lds_u32x4>(slot + fa.k[k + 2]);
      kb[k + 2] = *reinterpret_cast<lds_u32x4>(slot + fb.k[k + 2]);
    }
    sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka[k]), w.qf[k], sa, 0, 0, 0);
    sb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kb[k]), w.qf[k], sb, 0, 0, 0);
  }
  mask_scores(sa, la, hi);
  mask_scores(sb, lb, hi);
}

// The V^T fragment (A operand) of product (kk, dt) of a sub-block: two
// transposed reads of its 16-key group kk.
__device__ __forceinline__ bf16x8 vt_frag(const lds_u8* slot, const HFrag& f, int kk, int dt) {
  const lds_u8* vs = slot + kk * 16 * 256;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vs + f.v[dt]));
  const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vs + 8 * 256 + f.v[dt]));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ void sub_pv(const lds_u8* slot, const HFrag& f, const u32x4 (&pk)[2],
                                       WaveState& w) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      w.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt_frag(slot, f, kk, dt), as_bf16x8(pk[kk]),
                                                        w.o[dt], 0, 0, 0);
}

__device__ __forceinline__ void pack_probs(const float (&ps)[16], u32x4 (&pk)[2]) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int m = 0; m < 4; ++m) pk[kk][m] = pack_bf16x2(ps[8 * kk + 2 * m], ps[8 * kk + 2 * m + 1]);
}

// One step of one wave over its two 32-key sub-blocks, la and lb valid keys
// (as sub_scores' lim): the same online softmax as hstep, over 64 keys.
// Both sub-blocks are always computed: one code path per step keeps the
// accumulators in the same registers from step to step (a path that skips
// sub-block b makes the compiler move O between register sets every step).
// PAIR: the two sub-blocks' score products as interleaved chains with reads
// ahead (pair_scores); the dense walk keeps them as two chains, which it
// runs faster at long sequences (C5: 566 against 595 ms).
// qk_hook(k) runs between the score products (pair_scores_hooked).
template <bool PAIR = true, typename QKHook = NoHook>
__device__ __forceinline__ void sstep(const lds_u8* slot, const HFrag& fa, const HFrag& fb,
                                      float c, int la, int lb, int hi, WaveState& w,
                                      QKHook qk_hook = {}) {
  f32x16 sa, sb;
  if constexpr (!std::is_same<QKHook, NoHook>::value) {
    pair_scores_hooked(slot, fa, fb, w, la, lb, hi, sa, sb, qk_hook);
  } else if constexpr (PAIR) {
    pair_scores(slot, fa, fb, w, la, lb, hi, sa, sb);
  } else {
    sa = sub_scores(slot, fa, w, la, hi);
    sb = sub_scores(slot, fb, w, lb, hi);
  }

  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, sa[e]);
#pragma unroll
  for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, sb[e]);
  mloc = half_swap_max(mloc) * c;
  const float m_new = mloc > w.m_run + kRescaleSlack ? mloc : w.m_run;
  const float mu = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(w.m_run - mu);
  w.m_run = m_new;
  float pa[16], pb[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) pa[e] = __builtin_amdgcn_exp2f(fmaf(sa[e], c, -mu));
  float l4[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) l4[g] = (pa[4 * g] + pa[4 * g + 1]) + (pa[4 * g + 2] + pa[4 * g + 3]);
  float lsum = (l4[0] + l4[1]) + (l4[2] + l4[3]);
#pragma unroll
  for (int e = 0; e < 16; ++e) pb[e] = __builtin_amdgcn_exp2f(fmaf(sb[e], c, -mu));
#pragma unroll
  for (int g = 0; g < 4; ++g) l4[g] = (pb[4 * g] + pb[4 * g + 1]) + (pb[4 * g + 2] + pb[4 * g + 3]);
  lsum += (l4[0] + l4[1]) + (l4[2] + l4[3]);
  w.l_run = fmaf(w.l_run, alpha, lsum);
  u32x4 ka[2], kb[2];
  pack_probs(pa, ka);
  pack_probs(pb, kb);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) w.o[dt][e] *= alpha;
  }
  sub_pv(slot, fa, ka, w);
  sub_pv(slot, fb, kb, w);
}

// The step of a wave whose 32 query rows are all zero (the padding rows of
// a partial query tile, whose gathered q is zero): every valid key scores
// exactly 0, so P is 1 on the valid keys and 0 on the masked ones, the
// running max is 0 from the first valid key on and the row sum counts the
// valid keys. Only the P.V products remain; the result is bit-identical to
// sstep's on the same rows (the same products of the same exact P).
__device__ __forceinline__ void sstep_zero_q(const lds_u8* slot, const HFrag& fa,
                                             const HFrag& fb, int la, int lb, int hi,
                                             WaveState& w) {
  if (la <= 0 && lb <= 0) return;  // no valid key: P is 0 everywhere
  w.m_run = 0.f;
  auto probs = [&](int lim, u32x4 (&pk)[2]) {
    if (lim >= 32) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) pk[kk] = u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
      w.l_run += 16.f;
      return;
    }
    // register e holds key 8 (e / 4) + 4 hi + e % 4 of the sub-block
    float ps[16];
    int n = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const bool v = 8 * (e >> 2) + 4 * hi + (e & 3) < lim;
      ps[e] = v ? 1.f : 0.f;
      n += v;
    }
    w.l_run += (float)n;
    pack_probs(ps, pk);
  };
  u32x4 ka[2], kb[2];
  probs(la, ka);
  probs(lb, kb);
  sub_pv(slot, fa, ka, w);
  sub_pv(slot, fb, kb, w);
}

// Narrow walk (a query tile whose only real rows are its first 32): each
// wave takes one 32-key sub-block of every step, so the tile's products
// spread over all four SIMDs of the workgroup instead of one wave's chain.
// sstep_half is one sub-block (lim valid keys) of sstep for the tile's real
// rows, with hook(k) before the fragment reads of score product k + 2;
// sstep_half_zero is one sub-block of sstep_zero_q. The two sub-blocks'
// partial states are merged at the end of the walk.
template <typename Hook>
__device__ __forceinline__ void sstep_half(const lds_u8* slot, const HFrag& f, float c, int lim,
                                           int hi, WaveState& w, Hook hook) {
  typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
  f32x16 s;
#pragma unroll
  for (int e = 0; e < 16; ++e) s[e] = 0.f;
  u32x4 kf[8];
  kf[0] = *reinterpret_cast<lds_u32x4>(slot + f.k[0]);
  kf[1] = *reinterpret_cast<lds_u32x4>(slot + f.k[1]);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    hook(k);
    if (k + 2 < 8) kf[k + 2] = *reinterpret_cast<lds_u32x4>(slot + f.k[k + 2]);
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[k]), w.qf[k], s, 0, 0, 0);
  }
  mask_scores(s, lim, hi);
  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, s[e]);
  mloc = half_swap_max(mloc) * c;
  const float m_new = mloc > w.m_run + kRescaleSlack ? mloc : w.m_run;
  const float mu = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(w.m_run - mu);
  w.m_run = m_new;
  float ps[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) ps[e] = __builtin_amdgcn_exp2f(fmaf(s[e], c, -mu));
  float l4[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) l4[g] = (ps[4 * g] + ps[4 * g + 1]) + (ps[4 * g + 2] + ps[4 * g + 3]);
  w.l_run = fmaf(w.l_run, alpha, (l4[0] + l4[1]) + (l4[2] + l4[3]));
  u32x4 pk[2];
  pack_probs(ps, pk);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) w.o[dt][e] *= alpha;
  }
  sub_pv(slot, f, pk, w);
}

__device__ __forceinline__ void sstep_half_zero(const lds_u8* slot, const HFrag& f, int lim, int hi,
                                                WaveState& w) {
  if (lim <= 0) return;  // no valid key: P is 0 everywhere
  w.m_run = 0.f;
  u32x4 pk[2];
  if (lim >= 32) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) pk[kk] = u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    w.l_run += 16.f;
  } else {
    // register e holds key 8 (e / 4) + 4 hi + e % 4 of the sub-block
    float ps[16];
    int n = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const bool v = 8 * (e >> 2) + 4 * hi + (e & 3) < lim;
      ps[e] = v ? 1.f : 0.f;
      n += v;
    }
    w.l_run += (float)n;
    pack_probs(ps, pk);
  }
  sub_pv(slot, f, pk, w);
}

// The 16 weights of this lane's keys key0 + 8 g + 4 hi + m of a sub-block.
__device__ __forceinline__ void sub_weights(const uint8_t* wt, int key0, int hi, float (&ww)[16]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w4 = *reinterpret_cast<const uint32_t*>(wt + key0 + 8 * g + 4 * hi);
#pragma unroll
    for (int m = 0; m < 4; ++m) ww[4 * g + m] = (float)((w4 >> (8 * m)) & 0xffu);
  }
}

// A step of 64 virtual keys (the summaries of key tiles key0 .. key0 + 63)
// of the compensation of a given output: both sub-blocks' score products as
// interleaved chains (pair_scores, no key masked: virtual keys past n_k
// carry weight 0); then per sub-block p = exp2(s c - ref2) where the tile's
// weight (its real row count if dropped, else 0) is positive, den += p *
// weight, and O^T += V^T P^T, sub-block a's terms before b's.
//
// With the reference fixed, nothing of sub-block a waits for b's scores (no
// running max), so the step is software-pipelined: a's score products; b's
// score products with a's probabilities (vector unit) between them; a's
// P·V products with b's probabilities between them; b's P·V products. The
// matrix and vector units then work at once inside the wave instead of in
// turn. Every accumulator sees the same products in the same order as the
// plain sequence (a's scores, b's, a's P·V, b's), so the result is the
// same bit for bit.
__device__ __forceinline__ void vstep_fixed(const lds_u8* slot, const HFrag& fa, const HFrag& fb,
                                            float c, const uint8_t* wt, int key0, int hi,
                                            float ref2, WaveState& w) {
  typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
  // The order is written out, one product and its companions per stage,
  // with scheduling fences between the stages.
#define VEDA_FENCE() __builtin_amdgcn_sched_barrier(0)
  auto kread = [&](const HFrag& f, int k) { return *reinterpret_cast<lds_u32x4>(slot + f.k[k]); };
  // weights stay packed, four per word (byte m of word g is key 8 g + 4 hi + m)
  uint32_t wa[4], wb[4];
  auto wread = [&](int k0, uint32_t (&wp)[4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) wp[g] = *reinterpret_cast<const uint32_t*>(wt + k0 + 8 * g + 4 * hi);
  };
  f32x16 sa, sb;
#pragma unroll
  for (int e = 0; e < 16; ++e) sa[e] = sb[e] = 0.f;
  u32x4 ka[8], kb[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) ka[k] = kread(fa, k);
  VEDA_FENCE();
  // a's score products, K fragments read four ahead
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka[k]), w.qf[k], sa, 0, 0, 0);
    if (k < 4) ka[k + 4] = kread(fa, k + 4);
    else kb[k - 4] = kread(fb, k - 4);
    if (k == 0) wread(key0, wa);
    if (k == 1) wread(key0 + 32, wb);
    VEDA_FENCE();
  }
  // one sub-block's probabilities in eight pieces of two keys each (den
  // summed in key order, as in one pass)
  float den = 0.f;
  float ps[2];
  auto piece = [&](const f32x16& s, const uint32_t (&wp)[4], int k, u32x4 (&pk)[2]) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int e = 2 * k + m;
      const float ww = (float)((wp[e >> 2] >> (8 * (e & 3))) & 0xffu);
      const float x = ww > 0.f ? __builtin_amdgcn_exp2f(fmaf(s[e], c, -ref2)) : 0.f;
      ps[m] = x;
      den = fmaf(x, ww, den);
    }
    pk[k >> 2][k & 3] = pack_bf16x2(ps[0], ps[1]);
  };
  // b's score products with a's probabilities; a's first V^T fragments
  u32x4 pa[2], pb[2];
  bf16x8 va[2][4], vb[2][4];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kb[k]), w.qf[k], sb, 0, 0, 0);
    if (k < 4) kb[k + 4] = kread(fb, k + 4);
    else if (k < 6) va[0][k - 4] = vt_frag(slot, fa, 0, k - 4);
    piece(sa, wa, k, pa);
    VEDA_FENCE();
  }
  w.l_run += den;
  den = 0.f;
  // a's P.V products with b's probabilities, V^T fragments two ahead
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int kk = j >> 2, dt = j & 3;
    w.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[kk][dt], as_bf16x8(pa[kk]), w.o[dt], 0,
                                                      0, 0);
    const int n = j + 2;
    if (n < 8) va[n >> 2][n & 3] = vt_frag(slot, fa, n >> 2, n & 3);
    else vb[0][n - 8] = vt_frag(slot, fb, 0, n - 8);
    piece(sb, wb, j, pb);
    VEDA_FENCE();
  }
  w.l_run += den;
  // b's P.V products
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int kk = j >> 2, dt = j & 3;
    w.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb[kk][dt], as_bf16x8(pb[kk]), w.o[dt], 0,
                                                      0, 0);
    const int n = j + 2;
    if (n < 8) vb[n >> 2][n & 3] = vt_frag(slot, fb, n >> 2, n & 3);
    VEDA_FENCE();
  }
#undef VEDA_FENCE
}

// One sub-block (fragments f, first key k0) of virtual keys with the same
// probability x for every positive weight: den += x * weight and O^T +=
// V^T P^T, keys in the order vstep_fixed takes them.
__device__ __forceinline__ void vsub_const(const lds_u8* slot, const HFrag& f, const uint8_t* wt,
                                           int k0, int hi, float x, WaveState& w) {
  u32x4 pk[2];
  float den = 0.f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w4 = *reinterpret_cast<const uint32_t*>(wt + k0 + 8 * g + 4 * hi);
    float ps[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float ww = (float)((w4 >> (8 * m)) & 0xffu);
      ps[m] = ww > 0.f ? x : 0.f;
      den = fmaf(ps[m], ww, den);
    }
    pk[g >> 1][2 * (g & 1)] = pack_bf16x2(ps[0], ps[1]);
    pk[g >> 1][2 * (g & 1) + 1] = pack_bf16x2(ps[2], ps[3]);
  }
  w.l_run += den;
  sub_pv(slot, f, pk, w);
}

// vstep_fixed for a wave whose 32 query rows are all zero: every virtual
// key scores exactly 0, so p = exp2(-ref2) (x0, per row) wherever the
// key's weight is positive; only the P.V products remain. Same products,
// probabilities and den sums in the same order as vstep_fixed, so the
// result is the same bit for bit.
__device__ __forceinline__ void vstep_fixed_zero(const lds_u8* slot, const HFrag& fa,
                                                 const HFrag& fb, const uint8_t* wt, int key0,
                                                 int hi, float x0, WaveState& w) {
  vsub_const(slot, fa, wt, key0, hi, x0, w);
  vsub_const(slot, fb, wt, key0 + 32, hi, x0, w);
}

// vstep_fixed over one sub-block (fragments f, first key k0) for a narrow
// walk: its 8 score products, probabilities (den in vstep_fixed's key
// order) and 8 P.V products.
__device__ __forceinline__ void vstep_fixed_half(const lds_u8* slot, const HFrag& f, float c,
                                                 const uint8_t* wt, int k0, int hi, float ref2,
                                                 WaveState& w) {
  typedef const __attribute__((address_space(3))) u32x4* lds_u32x4;
  f32x16 s;
#pragma unroll
  for (int e = 0; e < 16; ++e) s[e] = 0.f;
  u32x4 kf[8];
  kf[0] = *reinterpret_cast<lds_u32x4>(slot + f.k[0]);
  kf[1] = *reinterpret_cast<lds_u32x4>(slot + f.k[1]);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k + 2 < 8) kf[k + 2] = *reinterpret_cast<lds_u32x4>(slot + f.k[k + 2]);
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf[k]), w.qf[k], s, 0, 0, 0);
  }
  u32x4 pk[2];
  float den = 0.f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w4 = *reinterpret_cast<const uint32_t*>(wt + k0 + 8 * g + 4 * hi);
    float ps[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float ww = (float)((w4 >> (8 * m)) & 0xffu);
      ps[m] = ww > 0.f ? __builtin_amdgcn_exp2f(fmaf(s[4 * g + m], c, -ref2)) : 0.f;
      den = fmaf(ps[m], ww, den);
    }
    pk[g >> 1][2 * (g & 1)] = pack_bf16x2(ps[0], ps[1]);
    pk[g >> 1][2 * (g & 1) + 1] = pack_bf16x2(ps[2], ps[3]);
  }
  w.l_run += den;
  sub_pv(slot, f, pk, w);
}

// One step of 64 virtual keys inside the online softmax (compensated
// attention): as sstep, with each key weighted by its tile's dropped
// real-row count (the denominator gains p * weight; the value is the
// tile's sum of V) and weight-0 keys masked out of the max.
__device__ __forceinline__ void sstep_virtual(const lds_u8* slot, const HFrag& fa,
                                              const HFrag& fb, float c, const uint8_t* wt,
                                              int key0, int hi, WaveState& w) {
  f32x16 sa = sub_scores(slot, fa, w, 32, hi);
  f32x16 sb = sub_scores(slot, fb, w, 32, hi);
  // weights stay packed, 4 per word (byte e % 4 of word e / 4 is key
  // 8 (e / 4) + 4 hi + e % 4 of the sub-block)
  uint32_t wa[4], wb[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    wa[g] = *reinterpret_cast<const uint32_t*>(wt + key0 + 8 * g + 4 * hi);
    wb[g] = *reinterpret_cast<const uint32_t*>(wt + key0 + 32 + 8 * g + 4 * hi);
  }
  auto byte = [](uint32_t x, int m) { return (x >> (8 * m)) & 0xffu; };
  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    sa[e] = byte(wa[e >> 2], e & 3) ? sa[e] : -INFINITY;
    sb[e] = byte(wb[e >> 2], e & 3) ? sb[e] : -INFINITY;
    mloc = fmaxf(mloc, fmaxf(sa[e], sb[e]));
  }
  mloc = half_swap_max(mloc) * c;
  const float m_new = mloc > w.m_run + kRescaleSlack ? mloc : w.m_run;
  const float mu = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(w.m_run - mu);
  w.m_run = m_new;
  float pa[16], pb[16], lsum = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    pa[e] = __builtin_amdgcn_exp2f(fmaf(sa[e], c, -mu));
    pb[e] = __builtin_amdgcn_exp2f(fmaf(sb[e], c, -mu));
    lsum = fmaf(pa[e], (float)byte(wa[e >> 2], e & 3), fmaf(pb[e], (float)byte(wb[e >> 2], e & 3), lsum));
  }
  w.l_run = fmaf(w.l_run, alpha, lsum);
  u32x4 ka[2], kb[2];
  pack_probs(pa, ka);
  pack_probs(pb, kb);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) w.o[dt][e] *= alpha;
  }
  sub_pv(slot, fa, ka, w);
  sub_pv(slot, fb, kb, w);
}

// Modes: kSparse walks the block lists. kVirtualOnly is the zero-order
// compensation of a given output: step u is virtual keys (tile summaries)
// 64 u .. 64 u + 63 of all n_k tiles, the reference is the row's fixed
// lse_kept instead of an online max, each key is weighted by its tile's
// dropped real-row count, and the epilogue adds o_kept and divides by
// 1 + den. kSparseComp is compensated attention in one pass: the list steps,
// then the virtual-key steps inside the same online softmax (a row that kept
// nothing first gets the reference's unit mass at reference 0, with value 0,
// so it ends as num / (1 + den) as well). kDenseRows is the dense forward
// of packed rows: step u is key rows 64 u .. of the `used` real rows (the
// last step clamped to them), and query rows at or past `used` get out 0
// and lse 0.
enum SparseMode { kSparse = 0, kVirtualOnly = 1, kSparseComp = 2, kDenseRows = 3 };

// SEQKV (kSparse in sequence order only): k and v are in sequence order too
// ([seq_rows, seq_heads_n, D], as q), and key tile row t of a step is read
// from row seq_q[t] of them (the gather of the key tiles fused into the
// walk).
template <int MODE, bool SEQKV = false>
__global__ void __launch_bounds__(kThreads2, 2) sfwd_kernel(FwdParams p) {
  constexpr bool DENSE = MODE == kDenseRows;
  constexpr bool LISTS = MODE == kSparse || MODE == kSparseComp;  // walks the block lists
  constexpr bool VKEYS = MODE == kVirtualOnly || MODE == kSparseComp;  // walks the virtual keys
  __shared__ __attribute__((aligned(1024))) uint8_t ring[2][kSlotBytes];
  __shared__ uint16_t steps[LISTS ? 2 * kMaxBlocks : 1];
  __shared__ uint8_t tvc[LISTS ? kMaxBlocks : 1];
  // virtual keys: per key tile, its real row count if dropped, else 0
  __shared__ __attribute__((aligned(16))) uint8_t vwt[VKEYS ? kMaxBlocks + kHalf : 4];
  __shared__ int32_t step_total, step_small, list_bad, list_unsorted;
  // sparse walk: which waves' 32 query rows are all zero, and the LSE of
  // their rows (all alike; see the copy waves below)
  __shared__ uint8_t zflag[4];
  __shared__ float zero_lse;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 31, hi = lane >> 5;
  int64_t head, r;
  front_first(blockIdx.x, p.n_heads, p.n_q_tiles, p.front, head, r);
  const int64_t qrow = r * kTile + 32 * wave + li;
  const int nk = (int)p.n_k_tiles;

  const int n_virt = VKEYS ? (nk + kHalf - 1) / kHalf : 0;
  const SDma cdma = sdma_offsets(VKEYS ? p.cs : 0, VKEYS ? p.cs : 0, wave, lane);  // summaries
  // Virtual step v: the summaries of key tiles 64 v .. 64 v + 63 (K and V
  // halves of the slot); in the last step rows past n_k do not exist, so
  // every lane reads a row below the step's count (the extra rows carry
  // weight 0).
  // load j of virtual step v: this wave's K segment j (j < 4) or V segment
  // j - 4
  auto virtual_seg = [&](int v, lds_u8* slot, int j) {
    const int64_t row0 = (int64_t)v * kHalf;
    const int vch = min(nk - v * kHalf, kHalf);
    const char* kb = reinterpret_cast<const char*>(p.kc + head * p.ch + row0 * p.cs);
    const char* vb = reinterpret_cast<const char*>(p.vc + head * p.ch + row0 * p.cs);
    const int u4 = j & 3, seg = 4 * wave + u4;
    lds_u8* dst = slot + (j < 4 ? 0 : kHalfBytes) + seg * 1024;
    if (vch == kHalf) {
      // cdma's offsets of waves 2, 3 count from row 32
      const int64_t sb = wave >= 2 ? 32 * p.cs * 2 : 0;
      dma16((j < 4 ? kb : vb) + sb, j < 4 ? cdma.k[u4] : cdma.v[u4], dst);
      return;
    }
    const int lr = lane >> 4, pc = lane & 15;
    const int row = 4 * seg + lr, src = min(row, vch - 1);
    const uint32_t off = j < 4 ? (uint32_t)((src * p.cs + ((pc ^ (row & 15)) << 3)) * 2)
                               : (uint32_t)((src * p.cs + ((pc ^ ((row & 3) << 2)) << 3)) * 2);
    dma16(j < 4 ? kb : vb, off, dst);
  };
  auto load_virtual = [&](int v, lds_u8* slot) {
#pragma unroll
    for (int j = 0; j < 8; ++j) virtual_seg(v, slot, j);
  };
  // Set-up: every independent global load goes out first (Q, the valid
  // counts, the list counts and the lists' first entries), so the set-up
  // waits for memory about once instead of once per dependent hop.
  WaveState w;
  const uint16_t* qptr = p.q + qrow * p.qs + head * p.qh;
  bool q_live = !DENSE || qrow < p.used;
  if (MODE == kSparse && p.seq_q != nullptr) {
    const int64_t sh = p.seq_heads[head], src = p.seq_q[qrow];
    q_live = p.slot_ok[qrow] != 0 && src >= 0 && src < p.seq_rows && sh >= 0 &&
             sh < p.seq_heads_n;
    qptr = p.q + (q_live ? src : 0) * p.qs + (q_live ? sh : 0) * p.qh;
  }
#pragma unroll
  for (int s = 0; s < 8; ++s)
    w.qf[s] = q_live ? as_bf16x8(ld16(qptr + 16 * s + 8 * hi)) : as_bf16x8(u32x4{0, 0, 0, 0});
  // compensation of a given output: the row's lse_kept, and the first
  // virtual step, which depends on nothing the set-up computes
  float lk = 0.f;
  if (MODE == kVirtualOnly) {
    lk = p.lse_kept[head * p.lk_h + qrow * p.lk_s];
    load_virtual(0, (lds_u8*)ring[0]);
  }
  if (VKEYS) {
    // weights of virtual keys 0 .. n_k - 1, padded with zeros to whole
    // steps, four per thread and word; both loads of an entry are issued
    // whatever its keep flag (indices clamped to n_k - 1), so the set-up
    // waits for memory once per pass instead of once per dependent load
    const uint8_t* keep_row = p.keep + (head * p.n_q_tiles + r) * p.n_k_tiles;
    for (int j4 = 4 * tid; j4 < n_virt * kHalf; j4 += 4 * kThreads2) {
      int kp[4], vn[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int jj = min(j4 + m, nk - 1);
        kp[m] = keep_row[jj];
        vn[m] = p.valid_count[jj];
      }
      uint32_t packed = 0;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int wj = (j4 + m < nk && kp[m] == 0) ? min(max(vn[m], 0), kTile) : 0;
        packed |= (uint32_t)wj << (8 * m);
      }
      *reinterpret_cast<uint32_t*>(vwt + j4) = packed;
    }
  }
  if (!LISTS) {
    if (tid == 0) step_total = DENSE ? (int)((p.used + kHalf - 1) / kHalf) : 0;
  } else {
    // Step list of 64-key halves (j << 2 | half << 1 | full), valid counts
    // in a byte table. A half with more than 32 valid keys (or a tile with
    // none: one void step) takes a step. Halves with 1..32 valid keys (the
    // ragged ends of partial tiles) are computed two to a step, one per
    // 32-key sub-block, so no step leaves a sub-block idle: the first of a
    // pair takes the step at its own place, flagged kPairStep, and the second
    // (its partner) is stored from the back of `steps` downwards, by pair
    // index.
    //
    // Walk order: the key tiles of both lists merged in ascending order,
    // starting at the first kept tile at or past tile r n_k / 512 (mod n_k)
    // and wrapping. The ~512 workgroups resident at once are consecutive
    // query tiles of a head, each started about 1/512 of a walk after the
    // previous one, so with this rotation they sweep the head's key tiles
    // together: a K/V line one of them fetches past L2 is more often still
    // there when the next workgroup of its XCD that keeps the tile reads it.
    // The rotation depends on the query tile alone, so the order (and the
    // summation order with it) is the same whichever heads a launch holds.
    // Lists that are not strictly ascending, share a tile, or hold an entry
    // outside [0, n_k) keep list order instead (the full list, then the
    // partial list, every entry as listed; an entry outside [0, n_k) is
    // void: two steps in the full list, one in the partial list).
    const int64_t li_ = head * p.n_q_tiles + r;
    const int ld = (int)p.list_ld;
    const int32_t* fl = p.full_idx + li_ * p.list_ld;
    const int32_t* pl = p.part_idx + li_ * p.list_ld;
    // the first entries of both lists, loaded before their counts arrive
    // (every row holds list_ld >= n_k entries)
    const int32_t f0 = tid < ld ? fl[tid] : -1;
    const int32_t p0 = tid < ld ? pl[tid] : -1;
    const int nf = min(max(p.full_cnt[li_], 0), min(ld, kMaxBlocks));
    const int np = min(max(p.part_cnt[li_], 0), min(ld, kMaxBlocks - nf));
    for (int j = tid; j < nk; j += kThreads2) tvc[j] = (uint8_t)min(max(p.valid_count[j], 0), kTile);
    // scratch in ring slot 1 (12 KB), which no load targets before the
    // walk's first barrier: both lists, then the walk order (j << 1 | full)
    uint16_t* sf = reinterpret_cast<uint16_t*>(&ring[1][0]);
    uint16_t* sp = sf + kMaxBlocks;
    uint16_t* sm = sp + kMaxBlocks;
    constexpr uint16_t kBadFull = 0xFFFF, kBadPart = 0xFFFE;  // entries outside [0, n_k)
    if (tid == 0) {
      list_bad = 0;
      list_unsorted = 0;
    }
    __syncthreads();  // valid counts in LDS, flags cleared
    bool bad = false;
    for (int i = tid; i < nf; i += kThreads2) {
      const int32_t j = i < kThreads2 ? f0 : fl[i];
      const bool ok = j >= 0 && j < nk;
      bad |= !ok;
      sf[i] = ok ? (uint16_t)j : kBadFull;
    }
    for (int i = tid; i < np; i += kThreads2) {
      const int32_t j = i < kThreads2 ? p0 : pl[i];
      const bool ok = j >= 0 && j < nk;
      bad |= !ok;
      sp[i] = ok ? (uint16_t)j : kBadPart;
    }
    if (bad) list_bad = 1;
    __syncthreads();  // both lists in LDS
    // entries of a[0, n) below `key` (a ascending)
    auto below = [](const uint16_t* a, int n, int key) {
      int lo = 0, up = n;
      while (lo < up) {
        const int mid = (lo + up) >> 1;
        if ((int)a[mid] < key)
          lo = mid + 1;
        else
          up = mid;
      }
      return lo;
    };
    if (__builtin_amdgcn_readfirstlane(list_bad) == 0) {
      // an entry's place in the merged order: its index plus the entries of
      // the other list with a lower tile
      bool uns = false;
      for (int i = tid; i < nf; i += kThreads2) {
        const int j = sf[i];
        const int k = below(sp, np, j);
        uns |= (i > 0 && sf[i - 1] >= j) || (k < np && sp[k] == j);
        sm[i + k] = (uint16_t)((j << 1) | 1);
      }
      for (int i = tid; i < np; i += kThreads2) {
        const int j = sp[i];
        const int k = below(sf, nf, j);
        uns |= (i > 0 && sp[i - 1] >= j) || (k < nf && sf[k] == j);
        sm[i + k] = (uint16_t)(j << 1);
      }
      if (uns) list_unsorted = 1;
    }
    __syncthreads();  // merged order (if the lists allow it)
    const bool sweep = __builtin_amdgcn_readfirstlane(list_bad | list_unsorted) == 0;
    if (!sweep) {
      for (int i = tid; i < nf; i += kThreads2)
        sm[i] = sf[i] == kBadFull ? kBadFull : (uint16_t)((sf[i] << 1) | 1);
      for (int i = tid; i < np; i += kThreads2)
        sm[nf + i] = sp[i] == kBadPart ? kBadPart : (uint16_t)(sp[i] << 1);
      __syncthreads();  // list order
    }
    if (wave == 0) {
      const int nm = nf + np;
      int m0 = 0;  // the walk's first entry
      if (sweep && nm > 0) {
        const int start = (int)((r * (int64_t)nk / kSweepWorkgroups) % nk);
        int lo = 0, up = nm;
        while (lo < up) {
          const int mid = (lo + up) >> 1;
          if ((int)(sm[mid] >> 1) < start)
            lo = mid + 1;
          else
            up = mid;
        }
        m0 = lo == nm ? 0 : lo;
      }
      // one entry per lane: its halves' steps at their places, from the
      // counts of big and ragged halves before them (ballots, so the order is
      // deterministic)
      int nbig = 0, nsm = 0;
      for (int q0 = 0; q0 < nm; q0 += 64) {
        const int q = q0 + lane;
        int m = q + m0;
        if (m >= nm) m -= nm;
        uint16_t e0 = kVoidStep, e1 = kVoidStep;
        bool b0 = false, r0 = false, b1 = false, r1 = false;  // big / ragged half 0, 1
        if (q < nm) {
          const uint16_t code = sm[m];
          if (code == kBadFull) {
            b0 = b1 = true;
          } else if (code == kBadPart) {
            b0 = true;
          } else {
            const int j = code >> 1;
            if (code & 1) {
              e0 = (uint16_t)((j << 2) | 1);
              e1 = (uint16_t)((j << 2) | 3);
              b0 = b1 = true;
            } else {
              const int vc = tvc[j];
              if (vc == 0) {
                b0 = true;  // no valid key: one void step
              } else {
                e0 = (uint16_t)(j << 2);
                b0 = min(vc, kHalf) > 32;
                r0 = !b0;
                if (vc > kHalf) {
                  e1 = (uint16_t)((j << 2) | 2);
                  b1 = vc - kHalf > 32;
                  r1 = !b1;
                }
              }
            }
          }
        }
        const int cb = (int)b0 + (int)b1, cr = (int)r0 + (int)r1;
        const uint64_t bb1 = __ballot(cb & 1), bb2 = __ballot(cb >> 1);
        const uint64_t br1 = __ballot(cr & 1), br2 = __ballot(cr >> 1);
        auto below_lane = [&](uint64_t b) {
          return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0));
        };
        const int B = nbig + below_lane(bb1) + 2 * below_lane(bb2);
        const int S = nsm + below_lane(br1) + 2 * below_lane(br2);
        // a big half's step follows the big halves and the pairs begun before it
        auto put = [&](uint16_t e, bool big, int bx, int sx) {
          if (big)
            steps[bx + ((sx + 1) >> 1)] = e;
          else if ((sx & 1) == 0)
            steps[bx + (sx >> 1)] = (uint16_t)(e | kPairStep);
          else
            steps[2 * kMaxBlocks - 1 - (sx >> 1)] = e;
        };
        if (b0 || r0) put(e0, b0, B, S);
        if (b1 || r1) put(e1, b1, B + (int)b0, S + (int)r0);
        nbig += __builtin_popcountll(bb1) + 2 * __builtin_popcountll(bb2);
        nsm += __builtin_popcountll(br1) + 2 * __builtin_popcountll(br2);
      }
      if (lane == 0) {
        step_total = nbig + (nsm + 1) / 2;
        step_small = nsm;
      }
    }
  }

#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" : : "v"(w.qf[s]));
  // a wave whose 32 query rows are all zero (padding rows) takes the
  // product-free step (wave-uniform)
  bool q_zero = false;
  if (MODE == kSparse || MODE == kSparseComp || MODE == kVirtualOnly) {
    uint32_t any = 0;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 x = __builtin_bit_cast(u32x4, w.qf[s]);
      any |= x[0] | x[1] | x[2] | x[3];
    }
    q_zero = __ballot(any != 0) == 0;
    if ((MODE == kSparse || MODE == kVirtualOnly) && lane == 0) zflag[wave] = q_zero ? 1 : 0;
    // wave 0's Q fragments for wave 1 of a narrow walk (below), in ring
    // slot 1 past the step-list scratch; no load reaches slot 1 before the
    // walk's first barrier
    if ((MODE == kSparse || MODE == kVirtualOnly) && wave == 0) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(
            (lds_u8*)ring[1] + kNarrowQ + (s * 64 + lane) * 16) = __builtin_bit_cast(u32x4, w.qf[s]);
    }
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) w.o[dt][e] = 0.f;
  w.m_run = -INFINITY;
  w.l_run = 0.f;
  // compensation of a given output: the row's fixed reference (0 for a row
  // that kept nothing)
  const float ref2 =
      MODE == kVirtualOnly && lk > -INFINITY && lk < INFINITY ? lk * 1.4426950408889634f : 0.f;
  __syncthreads();  // step list, weights, valid counts and list step count ready
  // All-zero query groups of one tile have the same output and LSE (the
  // uniform average over the tile's valid kept keys, the same products in
  // the same order): the first such wave computes it, the others ("copy"
  // waves) only load and pass the barriers, then store its staged rows.
  int zero_src = 0;
  bool copy = false, has_copy = false;  // has_copy: workgroup-uniform
  bool narrow = false;                  // workgroup-uniform
  if (MODE == kSparse) {
    const uint32_t zbits = __builtin_amdgcn_readfirstlane(
        (uint32_t)zflag[0] | ((uint32_t)zflag[1] << 1) | ((uint32_t)zflag[2] << 2) |
        ((uint32_t)zflag[3] << 3));
    zero_src = zbits ? __builtin_ctz(zbits) : 0;
    copy = q_zero && wave != zero_src;
    has_copy = __builtin_popcount(zbits) >= 2;
    narrow = zbits == 0xEu;
  }
  const int n_lsteps = __builtin_amdgcn_readfirstlane(step_total);
  // Narrow walk: only wave 0's rows are real (a tile with at most 32 valid
  // rows). Wave 0 takes sub-block a of every step and wave 1 sub-block b,
  // both for wave 0's rows (wave 1 takes wave 0's Q fragments from LDS);
  // waves 2 and 3 take the all-zero rows' products of sub-blocks a and b.
  // The halves merge after the walk; wave 2 then holds the all-zero rows'
  // output and waves 1 and 3 copy it.
  narrow = narrow && n_lsteps > 0;
  if (narrow) {
    zero_src = 2;
    copy = (wave & 1) != 0;
    if (wave == 1) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        w.qf[s] = as_bf16x8(*reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
            (const lds_u8*)ring[1] + kNarrowQ + (s * 64 + lane) * 16));
      // read before this wave reaches the walk's first barrier, after which
      // loads may target slot 1
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }
  const int n_small = LISTS ? __builtin_amdgcn_readfirstlane(step_small) : 0;
  const int n_steps = n_lsteps + n_virt;
  // Narrow compensation (a tile whose only real rows are wave 0's): waves 0
  // and 1 take wave 0's rows over sub-blocks a and b (wave 1 with wave 0's
  // Q fragments and references); waves 2 and 3 sum, over sub-blocks a and
  // b, the dropped tiles' V sums and weights that every all-zero row scales
  // by its own exp2(-ref2). Merged after the walk.
  bool vnarrow = false;
  float ref2_w = ref2;  // the reference of the rows this wave walks
  if (MODE == kVirtualOnly) {
    const uint32_t zbits = __builtin_amdgcn_readfirstlane(
        (uint32_t)zflag[0] | ((uint32_t)zflag[1] << 1) | ((uint32_t)zflag[2] << 2) |
        ((uint32_t)zflag[3] << 3));
    vnarrow = zbits == 0xEu && n_virt > 0;
    if (vnarrow && wave == 1) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        w.qf[s] = as_bf16x8(*reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
            (const lds_u8*)ring[1] + kNarrowQ + (s * 64 + lane) * 16));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // before slot 1 is loaded
      const float lk0 = p.lse_kept[head * p.lk_h + (r * kTile + li) * p.lk_s];
      ref2_w = lk0 > -INFINITY && lk0 < INFINITY ? lk0 * 1.4426950408889634f : 0.f;
    }
  }

  // Step u of the virtual and dense walks (the list walk decodes its own
  // steps): sub-block a is key rows row0 .. + 31 with la valid keys, sub-block
  // b rows rowb .. + 31 with lb (as sub_scores' lim). Steps n_lsteps .. are
  // virtual.
  auto decode = [&](int u, int64_t& row0, int& la, int64_t& rowb, int& lb) {
    if (VKEYS && u >= n_lsteps) {
      const int v = u - n_lsteps;
      row0 = (int64_t)v * kHalf;
      la = min(nk - v * kHalf, kHalf);
    } else if (DENSE) {
      row0 = (int64_t)u * kHalf;
      la = (int)min(p.used - row0, (int64_t)kHalf);
    } else {
      row0 = 0;
      la = 0;
    }
    rowb = row0 + 32;
    lb = la - 32;
  };
  const uint16_t* kbase = p.k + head * p.kh;
  const uint16_t* vbase = p.v + head * p.vh;
  const float c = p.scale_log2;
  const SDma dma = sdma_offsets(p.ks, p.vs, wave, lane);
  const HFrag fa = hfrag_offsets(0, lane), fb = hfrag_offsets(1, lane);
  const HFrag fh = hfrag_offsets(wave & 1, lane);  // a narrow walk's sub-block
  auto load_step = [&](int u, lds_u8* slot) {
    int64_t row0, rowb;
    int vch, lb;
    decode(u, row0, vch, rowb, lb);
    if (VKEYS && u >= n_lsteps) {
      load_virtual(u - n_lsteps, slot);
      return;
    }
    if (DENSE && vch < kHalf) {
      const char* kb = reinterpret_cast<const char*>(kbase + row0 * p.ks);
      const char* vb = reinterpret_cast<const char*>(vbase + row0 * p.vs);
      // the last dense step: rows past `used` may not exist, so every lane
      // reads a row below vch (masked keys)
      const int lr = lane >> 4, pc = lane & 15;
#pragma unroll
      for (int u4 = 0; u4 < 4; ++u4) {
        const int seg = 4 * wave + u4, row = 4 * seg + lr, src = min(row, vch - 1);
        const uint32_t ko = (uint32_t)((src * p.ks + ((pc ^ (row & 15)) << 3)) * 2);
        const uint32_t vo = (uint32_t)((src * p.vs + ((pc ^ ((row & 3) << 2)) << 3)) * 2);
        dma16(kb, ko, slot + seg * 1024);
        dma16(vb, vo, slot + kHalfBytes + seg * 1024);
      }
      return;
    }
    // waves 0, 1: sub-block a from row0; waves 2, 3: sub-block b from rowb.
    // Segments past a sub-block's valid keys reload its first rows (not
    // read: masked), so every wave issues the same loads.
    const bool wa = wave < 2;
    const int64_t base = wa ? row0 : rowb;
    const int lim = wa ? vch : lb + 32;
    const char* kb = reinterpret_cast<const char*>(kbase + base * p.ks);
    const char* vb = reinterpret_cast<const char*>(vbase + base * p.vs);
#pragma unroll
    for (int u4 = 0; u4 < 4; ++u4) {
      const int seg = 4 * wave + u4;
      const bool live = 4 * seg < lim;
      dma16(kb, live ? dma.k[u4] : dma.k_skip[u4], slot + seg * 1024);
      dma16(vb, live ? dma.v[u4] : dma.v_skip[u4], slot + kHalfBytes + seg * 1024);
    }
  };
  lds_u8* s0 = (lds_u8*)ring[0];
  lds_u8* s1 = (lds_u8*)ring[1];
  // Step u: wait for its own loads (the only ones in flight), barrier (all
  // waves' loads of step u are in LDS and all are done reading the other
  // slot), issue step u + 1 into the other slot, compute step u.
  // Compensation of a given output: o_kept's rows go to LDS as whole rows
  // during the last step (into the slot the epilogue stages the output in,
  // each wave its own 8 KB, with the output's layout) when every row start
  // is 16-byte aligned; otherwise the epilogue reads them itself.
  const bool kept_lds = MODE == kVirtualOnly &&
                        ((reinterpret_cast<uintptr_t>(p.o_kept) & 15) | ((p.oks | p.okh) & 7)) == 0;
  auto load_kept = [&](lds_u8* slot) {
    const char* kb = reinterpret_cast<const char*>(p.o_kept + (r * kTile + 32 * wave) * p.oks +
                                                   head * p.okh);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = 4 * i + (lane >> 4), ch = (lane & 15) ^ (rr & 15);
      dma16(kb, (uint32_t)((rr * p.oks + 8 * ch) * 2), slot + wave * 8192 + i * 1024);
    }
  };
  auto begin_step = [&](int u, lds_u8* nxt) {
    VEDA_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    if (u + 1 < n_steps)
      load_step(u + 1, nxt);
    else if (kept_lds)
      load_kept(nxt);
  };
  auto virtual_step = [&](int u, const lds_u8* cur) {
    // keys past n_k carry weight 0 (the table is padded), so no mask
    const int key0 = (u - n_lsteps) * kHalf;
    if (MODE == kVirtualOnly) {
      vstep_fixed(cur, fa, fb, c, vwt, key0, hi, ref2, w);
    } else {
      sstep_virtual(cur, fa, fb, c, vwt, key0, hi, w);
    }
  };
  if constexpr (MODE == kSparse || MODE == kSparseComp) {
    // Step records in registers: lane i of win_a / win_b holds sub-block a /
    // b of step 64 m + i of the current window m, as (first key row << 6 |
    // valid keys of the sub-block, clamped to 0 .. 32), decoded from the LDS
    // step list by all lanes at once, once per 64 steps. A step's record is
    // read into scalar registers (v_readlane) one step ahead, when its loads
    // are issued, and carried to its compute, so the loop itself reads no
    // step list and waits on no LDS read for it.
    uint32_t win_a = 0, win_b = 0;
    int pair_base = 0;  // pairs of ragged halves in the steps before the window
    auto lane_half = [&](int e, int64_t& r0, int& vch) {
      if (e == kVoidStep) {
        r0 = 0;
        vch = 0;
        return;
      }
      const int j = e >> 2, half = (e >> 1) & 1, full = e & 1;
      const int vc = full ? kTile : (int)tvc[j];
      r0 = (int64_t)j * kTile + half * kHalf;
      vch = half ? vc - kHalf : min(vc, kHalf);
    };
    // (windows are refilled in step order, so pair_base counts the pairs
    // before each window)
    auto refill = [&](int base) {
      const int u = base + lane;
      const bool in = u < n_lsteps;
      const int e = in ? (int)steps[u] : (int)kVoidStep;
      const bool pair = in && e != kVoidStep && (e & kPairStep) != 0;
      const uint64_t bp = __ballot(pair);
      const int k = pair_base + __builtin_amdgcn_mbcnt_hi(
                                    (uint32_t)(bp >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bp, 0));
      pair_base += __builtin_popcountll(bp);
      int64_t row0 = 0, rowb = 0;
      int la = 0, lb = 0;
      if (pair) {
        lane_half(e & ~(int)kPairStep, row0, la);
        // the last ragged half of an odd count has no partner: sub-block b
        // loads sub-block a's rows (a kept tile), all of them masked
        rowb = row0;
        if (2 * k + 1 < n_small) lane_half(steps[2 * kMaxBlocks - 1 - k], rowb, lb);
      } else if (in) {
        lane_half(e, row0, la);
        rowb = row0 + 32;
        lb = la - 32;
      }
      win_a = ((uint32_t)row0 << 6) | (uint32_t)min(max(la, 0), 32);
      win_b = ((uint32_t)rowb << 6) | (uint32_t)min(max(lb, 0), 32);
    };
    auto fetch = [&](int u, uint32_t& ra, uint32_t& rb) {
      if ((u & 63) == 0) refill(u);
      ra = (uint32_t)__builtin_amdgcn_readlane((int)win_a, u & 63);
      rb = (uint32_t)__builtin_amdgcn_readlane((int)win_b, u & 63);
    };
    // A step's loads: waves 0, 1 load sub-block a, waves 2, 3 sub-block b,
    // rows 16 (wave & 1) .. + 15 of it as four 1 KB segments of K and four of
    // V, with no branch. Segments past the sub-block's valid keys load the
    // key tile's own padding rows, as the reference's kernel reads them (they
    // are masked: the scores become -inf, the probabilities exactly 0); at
    // C2 they are 0.5 % of the segments.
    auto rec_base = [&](uint32_t ra, uint32_t rb, const char*& kb, const char*& vb) {
      const int64_t base = (int64_t)((wave < 2 ? ra : rb) >> 6);
      kb = reinterpret_cast<const char*>(kbase + base * p.ks);
      vb = reinterpret_cast<const char*>(vbase + base * p.vs);
    };
    // load j of a step: K segment j (j < 4) or V segment j - 4, into the
    // slot whose segment 4 wave (this wave's first) is at LDS address lds
    auto issue = [&](const char* kb, const char* vb, int j, uint32_t lds) {
      const int u4 = j & 3;
      if (j < 4)
        dma16_m0(kb, dma.k[u4], lds + u4 * 1024);
      else
        dma16_m0(vb, dma.v[u4], lds + kHalfBytes + u4 * 1024);
    };
    // this wave's first segment of each slot, as LDS addresses
    const uint32_t lds_s0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(s0 + 4 * wave * 1024));
    const uint32_t lds_s1 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(s1 + 4 * wave * 1024));
    // Step (ra, rb) from `cur`, with the loads of step (na, nb) into `nxt`
    // (unless it is the last step) issued between its products, so a load
    // that waits for the CU's load path waits beside this wave's own running
    // products. Issued in one burst after the barrier, the loads of all
    // eight waves of a CU queue at the load path together and each wave
    // stalls on them.
    // kind: 0 a wave with a real query row, 1 the wave that computes the
    // all-zero groups' output, 2 a copy wave (loads only); in a narrow
    // walk, 3 a wave with the tile's real rows over one sub-block and 4 the
    // all-zero rows over one sub-block
    // Compensated attention: the last list step loads the first virtual
    // step (the tile summaries) instead.
    const bool virt_next = MODE == kSparseComp && n_virt > 0;
    auto step = [&](auto kind, bool more, uint32_t ra, uint32_t rb, const lds_u8* cur,
                    uint32_t na, uint32_t nb, uint32_t nxt, lds_u8* nxt_slot)
        __attribute__((always_inline)) {
      const int la = (int)(ra & 63u), lb = (int)(rb & 63u);
      const char *kb, *vb;
      rec_base(na, nb, kb, vb);
      if constexpr (decltype(kind)::value == 3) {
        sstep_half(cur, fh, c, (wave & 1) ? lb : la, hi, w, [&](int k) {
          if (more) issue(kb, vb, k, nxt);
        });
      } else if constexpr (decltype(kind)::value != 0) {
        if (more) {
#pragma unroll
          for (int j = 0; j < 8; ++j) issue(kb, vb, j, nxt);
        } else if (virt_next) {
#pragma unroll
          for (int j = 0; j < 8; ++j) virtual_seg(0, nxt_slot, j);
        }
        if constexpr (decltype(kind)::value == 1) sstep_zero_q(cur, fa, fb, la, lb, hi, w);
        if constexpr (decltype(kind)::value == 4) sstep_half_zero(cur, fh, (wave & 1) ? lb : la, hi, w);
      } else {
        sstep(cur, fa, fb, c, la, lb, hi, w, [&](int k) {
          if (more) issue(kb, vb, k, nxt);
          else if (virt_next) virtual_seg(0, nxt_slot, k);
        });
      }
    };
    // A copy of the walk per kind of wave (same loads and barriers), so
    // each keeps O in one set of registers. Step u computes from slot u % 2
    // and loads step u + 1 into the other.
    auto walk = [&](auto zero) __attribute__((always_inline)) {
      uint32_t ca = 0, cb = 0;
      if (n_lsteps > 0) {
        fetch(0, ca, cb);
        const char *kb, *vb;
        rec_base(ca, cb, kb, vb);
#pragma unroll
        for (int j = 0; j < 8; ++j) issue(kb, vb, j, lds_s0);
      } else if (virt_next) {
        load_virtual(0, s0);
      }
      for (int u = 0; u < n_lsteps; u += 2) {
        uint32_t na = 0, nb = 0;
        VEDA_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        const bool more1 = u + 1 < n_lsteps;
        if (more1) fetch(u + 1, na, nb);
        step(zero, more1, ca, cb, s0, na, nb, lds_s1, s1);
        if (!more1) break;
        VEDA_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        const bool more2 = u + 2 < n_lsteps;
        if (more2) fetch(u + 2, ca, cb);
        step(zero, more2, na, nb, s1, ca, cb, lds_s0, s0);
      }
    };
    // Sequence-order k / v: this wave's four segments of a step are rows
    // 16 (wave & 1) + 4 u4 + lane / 16 of its sub-block; each is read from
    // the row its slot gathers (the low word of the int64 gather index),
    // and a row past the sub-block's valid keys (padding, masked) from the
    // sub-block's first row, a real row of the same key tile (so a
    // non-finite value there reaches only query tiles that keep the block,
    // as in the tiled form). The rows of step u + 2 are looked up during
    // step u, so the step's loads wait for no lookup.
    const int32_t* tok_of = reinterpret_cast<const int32_t*>(p.seq_q);
    const int kv_head = SEQKV ? (int)min(max(p.seq_heads[head], (int64_t)0), p.seq_heads_n - 1) : 0;
    const char* kseq = reinterpret_cast<const char*>(p.k + (int64_t)kv_head * p.kh);
    const char* vseq = reinterpret_cast<const char*>(p.v + (int64_t)kv_head * p.vh);
    auto tokens = [&](uint32_t ra, uint32_t rb, int32_t (&t)[4]) {
      const uint32_t rec = wave < 2 ? ra : rb;
      const int64_t base = (int64_t)(rec >> 6);
      const int lim = (int)(rec & 63u);
#pragma unroll
      for (int u4 = 0; u4 < 4; ++u4) {
        const int src = 16 * (wave & 1) + 4 * u4 + (lane >> 4);
        t[u4] = tok_of[2 * (base + (src < lim ? src : 0))];
      }
    };
    // byte offset of a row: row * (2 stride_s) fits 32 bits (the launcher
    // checks), k and v share the stride; the chunk swizzles of the slot rows
    // are per-lane constants
    const uint32_t row_bytes = (uint32_t)(2 * p.ks);
    const uint32_t n_rows = (uint32_t)p.seq_rows;
    uint32_t kswz[4], vswz[4];
#pragma unroll
    for (int u4 = 0; u4 < 4; ++u4) {
      const int pc = lane & 15, row = 4 * (4 * wave + u4) + (lane >> 4);  // slot row
      kswz[u4] = (uint32_t)((pc ^ (row & 15)) << 4);
      vswz[u4] = (uint32_t)((pc ^ ((row & 3) << 2)) << 4);
    }
    auto offsets = [&](const int32_t (&t)[4], uint32_t (&ok)[4], uint32_t (&ov)[4]) {
#pragma unroll
      for (int u4 = 0; u4 < 4; ++u4) {
        const uint32_t tk = (uint32_t)t[u4] < n_rows ? (uint32_t)t[u4] : 0u;
        const uint32_t b = tk * row_bytes;
        ok[u4] = b + kswz[u4];
        ov[u4] = b + vswz[u4];
      }
    };
    auto issue_kv = [&](const uint32_t (&ok)[4], const uint32_t (&ov)[4], int j, uint32_t lds) {
      const int u4 = j & 3;
      if (j < 4)
        dma16_m0(kseq, ok[u4], lds + u4 * 1024);
      else
        dma16_m0(vseq, ov[u4], lds + kHalfBytes + u4 * 1024);
    };
    auto step_kv = [&](auto kind, bool more, uint32_t ra, uint32_t rb, const lds_u8* cur,
                       const uint32_t (&ok)[4], const uint32_t (&ov)[4], uint32_t nxt)
        __attribute__((always_inline)) {
      const int la = (int)(ra & 63u), lb = (int)(rb & 63u);
      if constexpr (decltype(kind)::value == 3) {
        sstep_half(cur, fh, c, (wave & 1) ? lb : la, hi, w, [&](int k) {
          if (more) issue_kv(ok, ov, k, nxt);
        });
      } else if constexpr (decltype(kind)::value != 0) {
        if (more) {
#pragma unroll
          for (int j = 0; j < 8; ++j) issue_kv(ok, ov, j, nxt);
        }
        if constexpr (decltype(kind)::value == 1) sstep_zero_q(cur, fa, fb, la, lb, hi, w);
        if constexpr (decltype(kind)::value == 4) sstep_half_zero(cur, fh, (wave & 1) ? lb : la, hi, w);
      } else {
        sstep(cur, fa, fb, c, la, lb, hi, w, [&](int k) {
          if (more) issue_kv(ok, ov, k, nxt);
        });
      }
    };
    // the walk above with sequence-order k / v; (ra0, rb0) and (ra1, rb1)
    // are the records of steps u and u + 1, tk the rows of the next step
    // whose loads are not issued yet
    auto walk_kv = [&](auto zero) __attribute__((always_inline)) {
      uint32_t ra0 = 0, rb0 = 0, ra1 = 0, rb1 = 0;
      int32_t tk[4] = {0, 0, 0, 0};
      uint32_t ok[4], ov[4];
      if (n_lsteps > 0) {
        fetch(0, ra0, rb0);
        tokens(ra0, rb0, tk);
        offsets(tk, ok, ov);
#pragma unroll
        for (int j = 0; j < 8; ++j) issue_kv(ok, ov, j, lds_s0);
      }
      if (n_lsteps > 1) {
        fetch(1, ra1, rb1);
        tokens(ra1, rb1, tk);
      }
      for (int u = 0; u < n_lsteps; u += 2) {
        VEDA_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        const bool more1 = u + 1 < n_lsteps;
        uint32_t ra2 = 0, rb2 = 0;
        if (more1) offsets(tk, ok, ov);  // step u + 1
        if (u + 2 < n_lsteps) {
          fetch(u + 2, ra2, rb2);
          tokens(ra2, rb2, tk);
        }
        step_kv(zero, more1, ra0, rb0, s0, ok, ov, lds_s1);
        if (!more1) break;
        VEDA_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        const bool more2 = u + 2 < n_lsteps;
        uint32_t ra3 = 0, rb3 = 0;
        if (more2) offsets(tk, ok, ov);  // step u + 2
        if (u + 3 < n_lsteps) {
          fetch(u + 3, ra3, rb3);
          tokens(ra3, rb3, tk);
        }
        step_kv(zero, more2, ra1, rb1, s1, ok, ov, lds_s0);
        ra0 = ra2;
        rb0 = rb2;
        ra1 = ra3;
        rb1 = rb3;
      }
    };
    if constexpr (SEQKV) {
      if (narrow && wave < 2)
        walk_kv(std::integral_constant<int, 3>{});
      else if (narrow)
        walk_kv(std::integral_constant<int, 4>{});
      else if (copy)
        walk_kv(std::integral_constant<int, 2>{});
      else if (q_zero)
        walk_kv(std::integral_constant<int, 1>{});
      else
        walk_kv(std::integral_constant<int, 0>{});
    } else {
      if (narrow && wave < 2)
        walk(std::integral_constant<int, 3>{});
      else if (narrow)
        walk(std::integral_constant<int, 4>{});
      else if (copy)
        walk(std::integral_constant<int, 2>{});
      else if (q_zero)
        walk(std::integral_constant<int, 1>{});
      else
        walk(std::integral_constant<int, 0>{});
    }
    if constexpr (MODE == kSparseComp) {
      // a row that kept nothing: the reference's unit mass at reference 0
      // (a select, not a branch: the condition is per row)
      const bool empty = half_swap_sum(w.l_run) == 0.f;
      w.m_run = empty ? 0.f : w.m_run;
      w.l_run = empty ? (hi == 0 ? 1.f : 0.f) : w.l_run;
      // the virtual steps: step u from slot u % 2 (the first one's loads
      // were issued by the last list step, or above), each issuing the next
      int u = n_lsteps;
      if (u & 1) {
        if (u < n_steps) {
          begin_step(u, s0);
          virtual_step(u, s1);
          ++u;
        }
      }
      for (; u + 1 < n_steps; u += 2) {
        begin_step(u, s1);
        virtual_step(u, s0);
        begin_step(u + 1, s0);
        virtual_step(u + 1, s1);
      }
      if (u < n_steps) {
        begin_step(u, s1);
        virtual_step(u, s0);
      }
    }
  } else {
  if (n_steps > 0 && MODE != kVirtualOnly) load_step(0, s0);  // kVirtualOnly: issued at set-up
  if constexpr (DENSE) {
    // Dense walk: step u is key rows 64 u .. of the used rows, from slot
    // u % 2. It waits for its own loads and passes the barrier, then issues
    // step u + 1's loads between its score products (as the sparse walk
    // does), the last step's rows clamped to the used ones.
    auto dstep = [&](int u, const lds_u8* cur, lds_u8* nxt) {
      VEDA_WAIT_VM(0);
      __builtin_amdgcn_s_barrier();
      const bool more = u + 1 < n_steps;
      const int64_t row0 = (int64_t)u * kHalf;
      const int vch = (int)min(p.used - row0, (int64_t)kHalf);
      const int64_t nrow0 = row0 + kHalf;
      const int nvch = more ? (int)min(p.used - nrow0, (int64_t)kHalf) : 0;
      // waves 0, 1 load sub-block a, waves 2, 3 sub-block b (rows from 32)
      const int64_t nbase = nvch == kHalf && wave >= 2 ? nrow0 + 32 : nrow0;
      const char* kb = reinterpret_cast<const char*>(kbase + nbase * p.ks);
      const char* vb = reinterpret_cast<const char*>(vbase + nbase * p.vs);
      const int lr = lane >> 4, pc = lane & 15;
      auto hook = [&](int j) {
        if (!more) return;
        const int u4 = j & 3, seg = 4 * wave + u4;
        lds_u8* dst = nxt + (j < 4 ? 0 : kHalfBytes) + seg * 1024;
        if (nvch == kHalf) {
          dma16(j < 4 ? kb : vb, j < 4 ? dma.k[u4] : dma.v[u4], dst);
        } else {
          // the last step: rows past `used` may not exist, so every lane
          // reads a row below nvch (masked keys)
          const int row = 4 * seg + lr, src = min(row, nvch - 1);
          const uint32_t off = j < 4 ? (uint32_t)((src * p.ks + ((pc ^ (row & 15)) << 3)) * 2)
                                     : (uint32_t)((src * p.vs + ((pc ^ ((row & 3) << 2)) << 3)) * 2);
          dma16(j < 4 ? kb : vb, off, dst);
        }
      };
      sstep(cur, fa, fb, c, vch, vch - 32, hi, w, hook);
    };
    for (int u = 0; u < n_steps; u += 2) {
      dstep(u, s0, s1);
      if (u + 1 >= n_steps) break;
      dstep(u + 1, s1, s0);
    }
  } else {
    // compensation of a given output: the virtual steps, step u in slot
    // u % 2 (step 0's loads went out at set-up), unrolled by two so that
    // every fragment read has a constant slot address. A wave whose 32
    // query rows are all zero takes the product-free step (one copy of the
    // loop per kind, so O stays in one set of registers).
    auto vwalk = [&](auto zero) __attribute__((always_inline)) {
      const float x0 = __builtin_amdgcn_exp2f(-ref2);
      auto vstep = [&](int v, const lds_u8* cur) __attribute__((always_inline)) {
        constexpr int K = decltype(zero)::value;
        const int k0 = v * kHalf + 32 * (wave & 1);  // a narrow walk's sub-block
        if constexpr (K == 1)
          vstep_fixed_zero(cur, fa, fb, vwt, v * kHalf, hi, x0, w);
        else if constexpr (K == 2)
          vstep_fixed_half(cur, fh, c, vwt, k0, hi, ref2_w, w);
        else if constexpr (K == 3)
          vsub_const(cur, fh, vwt, k0, hi, 1.f, w);
        else
          virtual_step(v, cur);
      };
      int u = 0;
      for (; u + 1 < n_steps; u += 2) {
        begin_step(u, s1);
        vstep(u, s0);
        begin_step(u + 1, s0);
        vstep(u + 1, s1);
      }
      if (u < n_steps) {
        begin_step(u, s1);
        vstep(u, s0);
      }
    };
    if (MODE == kVirtualOnly && vnarrow)
      wave < 2 ? vwalk(std::integral_constant<int, 2>{}) : vwalk(std::integral_constant<int, 3>{});
    else if (MODE == kVirtualOnly && q_zero)
      vwalk(std::integral_constant<int, 1>{});
    else
      vwalk(std::integral_constant<int, 0>{});
  }
  }  // the dense walk and the compensation of a given output

  if (MODE == kVirtualOnly && vnarrow) {
    // Merge the narrow compensation: wave 1's sums (wave 0's rows over
    // sub-block b, against the same fixed references) into wave 0's; wave 3's
    // V sum and weights (all columns alike; lanes 0 and 32 pass them) into
    // wave 2's, which then hands the totals S and W to waves 1 to 3: an
    // all-zero row with p = x0 = exp2(-ref2) on every positive weight has
    // O = bf16(x0) S and den = x0 W. Through the last step's slot once every
    // wave is done with it (the other slot holds the o_kept rows).
    float* xo = reinterpret_cast<float*>(ring[(n_steps - 1) & 1]);
    float* xz = xo + 65 * 64;
    float* xs = xz + 132;
    __syncthreads();
    if (wave == 1) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) xo[(16 * dt + e) * 64 + lane] = w.o[dt][e];
      xo[64 * 64 + lane] = w.l_run;
    } else if (wave == 3 && li == 0) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) xz[(16 * dt + e) * 2 + hi] = w.o[dt][e];
      xz[128 + hi] = w.l_run;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) w.o[dt][e] += xo[(16 * dt + e) * 64 + lane];
      w.l_run += xo[64 * 64 + lane];
    } else if (wave == 2 && li == 0) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          xs[(16 * dt + e) * 2 + hi] = w.o[dt][e] + xz[(16 * dt + e) * 2 + hi];
      xs[128 + hi] = w.l_run + xz[128 + hi];
    }
    __syncthreads();
    if (wave != 0) {
      const float x0 = __builtin_amdgcn_exp2f(-ref2);
      const float xb = bf16_to_f32(pack_bf16x2(x0, 0.f) & 0xffffu);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) w.o[dt][e] = xb * xs[(16 * dt + e) * 2 + hi];
      w.l_run = x0 * xs[128 + hi];
    }
  }

  if (MODE == kSparse && narrow) {
    // Merge the narrow walk's halves: wave 1's state (the real rows over
    // sub-block b) into wave 0's, wave 3's (the all-zero rows over b) into
    // wave 2's, through the last step's slot once every wave is done with
    // it. Lane l of a pair holds the same row and keys on both sides;
    // each side's O and l are relative to its own reference m, so both
    // move to the larger one (a side with no valid key has m = -inf and
    // weighs 0). The zero rows' state is the same for every row, so wave 3
    // passes one row's (lanes 0 and 32).
    float* xo = reinterpret_cast<float*>(ring[(n_steps - 1) & 1]);
    float* xz = xo + 66 * 64;
    __syncthreads();
    if (wave == 1) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) xo[(16 * dt + e) * 64 + lane] = w.o[dt][e];
      xo[64 * 64 + lane] = w.m_run;
      xo[65 * 64 + lane] = w.l_run;
    } else if (wave == 3 && li == 0) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) xz[(16 * dt + e) * 2 + hi] = w.o[dt][e];
      xz[128 + hi] = w.m_run;
      xz[130 + hi] = w.l_run;
    }
    __syncthreads();
    if (wave == 0 || wave == 2) {
      const int ix = wave == 0 ? lane : hi, n = wave == 0 ? 64 : 2;
      const float* src = wave == 0 ? xo : xz;
      const float mb = src[64 * n + ix], lb = src[65 * n + ix];
      const float m = fmaxf(w.m_run, mb);
      const float mu = m == -INFINITY ? 0.f : m;
      const float aa = __builtin_amdgcn_exp2f(w.m_run - mu), ab = __builtin_amdgcn_exp2f(mb - mu);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) w.o[dt][e] = w.o[dt][e] * aa + src[(16 * dt + e) * n + ix] * ab;
      w.l_run = w.l_run * aa + lb * ab;
      w.m_run = m;
    }
  }

  const float l = half_swap_sum(w.l_run);
  // compensation: the kept output is num / den over the kept keys with
  // den = 1 at the reference, hence out = (o_kept + num) / (1 + den)
  const bool row_real = !DENSE || qrow < p.used;
  const float inv = MODE == kVirtualOnly ? 1.f / (1.f + l) : (l > 0.f && row_real) ? 1.f / l : 0.f;
  const bool row_exists = !DENSE || qrow < p.q_rows;  // rows past seq_len do not exist
  uint16_t* orow = p.out + (row_exists ? qrow : 0) * p.os + head * p.oh;
  bool o_live = row_exists;
  if (MODE == kSparse && p.seq_o != nullptr) {
    const int64_t sh = p.seq_heads[head], dst = p.seq_o[qrow];
    o_live = p.slot_ok[qrow] != 0 && dst >= 0 && dst < p.out_rows && sh >= 0 &&
             sh < p.seq_heads_n;
    orow = p.out + (o_live ? dst : 0) * p.os + (o_live ? sh : 0) * p.oh;
  }
  const uint16_t* krow = MODE == kVirtualOnly ? p.o_kept + qrow * p.oks + head * p.okh : nullptr;
  // The output goes out as whole rows: each wave writes its 32 rows (bf16)
  // into its 8 KB of the slot no step reads any more (the last step's is
  // n_steps - 1's; every wave has passed the barrier after step n_steps - 2,
  // which used this one), 16-byte chunk c of row r at c ^ (r % 16), then
  // lane l stores chunk l % 16 of rows 4 i + l / 16: four rows per store
  // instead of 16 bytes of each of 32 rows.
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  lds_u8* stage = (lds_u8*)ring[n_steps & 1] + wave * 8192;
  if (kept_lds) VEDA_WAIT_VM(0);  // this wave's o_kept rows are in its part of `stage`
  if (!copy) {
    // compensation: all 16 pieces of o_kept are read before any is used
    // (one wait instead of one per piece)
    u32x2 kv[4][4];
    if (MODE == kVirtualOnly) {
      if (kept_lds) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            kv[dt][g] = *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(
                stage + li * 256 + (((4 * dt + g) ^ (li & 15)) << 4) + 8 * hi);
      } else {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            kv[dt][g] = *reinterpret_cast<const u32x2*>(krow + 32 * dt + 8 * g + 4 * hi);
      }
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int e = 4 * g;
        float kept4[4] = {0.f, 0.f, 0.f, 0.f};
        if (MODE == kVirtualOnly) {
          kept4[0] = bf16_to_f32(kv[dt][g][0] & 0xffffu);
          kept4[1] = bf16_to_f32(kv[dt][g][0] >> 16);
          kept4[2] = bf16_to_f32(kv[dt][g][1] & 0xffffu);
          kept4[3] = bf16_to_f32(kv[dt][g][1] >> 16);
        }
        float v4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          v4[m] = (MODE == kVirtualOnly ? kept4[m] + w.o[dt][e + m] : w.o[dt][e + m]) * inv;
        const uint32_t w0 = pack_bf16x2(v4[0], v4[1]), w1 = pack_bf16x2(v4[2], v4[3]);
        *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(
            stage + li * 256 + (((4 * dt + g) ^ (li & 15)) << 4) + 8 * hi) = u32x2{w0, w1};
      }
  }
  float lse_val = !row_real ? 0.f : l > 0.f ? (w.m_run + __log2f(l)) * kLn2 : -INFINITY;
  const lds_u8* src = stage;
  if (has_copy) {
    // copy waves store the rows (and LSE) the first all-zero wave staged
    if (wave == zero_src && lane == 0) zero_lse = lse_val;
    __syncthreads();
    if (copy) {
      src = (const lds_u8*)ring[n_steps & 1] + zero_src * 8192;
      lse_val = zero_lse;
    }
  }
  asm volatile("" ::: "memory");
  const uint64_t orow_bits = reinterpret_cast<uintptr_t>(orow);
  const bool row16 = ((p.os | p.oh) & 7) == 0;  // every row start 16-byte aligned
  // rows in sequence order come from the lane that owns the row; otherwise
  // row rr of this wave's 32 is at a fixed stride
  const bool seq_rows = MODE == kSparse && p.seq_o != nullptr;
  uint16_t* const wave_rows = p.out + (r * kTile + 32 * wave) * p.os + head * p.oh;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int rr = 4 * i + (lane >> 4), ch = lane & 15;
    const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
        src + rr * 256 + ((ch ^ (rr & 15)) << 4));
    uint16_t* dst;
    bool live;
    if (seq_rows) {
      const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)orow_bits, rr);
      const uint32_t up = (uint32_t)__shfl((int)(uint32_t)(orow_bits >> 32), rr);
      live = __shfl((int)o_live, rr) != 0;
      dst = reinterpret_cast<uint16_t*>((uintptr_t)(((uint64_t)up << 32) | lo)) + 8 * ch;
    } else {
      live = !DENSE || r * kTile + 32 * wave + rr < p.q_rows;
      dst = wave_rows + rr * p.os + 8 * ch;
    }
    if (live) {
      if (row16) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {  // rows 8-byte aligned only (strides that are multiples of 4 elements)
        *reinterpret_cast<u32x2*>(dst) = u32x2{v[0], v[1]};
        *reinterpret_cast<u32x2*>(dst + 4) = u32x2{v[2], v[3]};
      }
    }
  }
  if ((MODE == kSparse || DENSE) && p.lse != nullptr && hi == 0 && row_exists)
    p.lse[head * p.lse_sh + qrow * p.lse_ss] = lse_val;
}

// ---------------------------------------------------------------------------
// Teacher statistics pass (no dense output): the LSE of every query row over
// all valid keys, and per (key tile, row) the block statistic of the heat.
//
// Workgroup = (head, group of four query items), 16 waves, so each K tile
// fetched into LDS serves four query tiles. Wave w owns item w / 4 of the
// group, rows 32 (w % 4) .. + 31 (Q^T in registers), and all 64 keys of every
// step (two 32-key sub-blocks): the same online softmax as the sparse
// forward's (log2 domain, reference max raised only past a slack of 8), with
// the current key tile's partial (sum relative to the reference, or the raw
// max) in a register, written as one log2 statistic per row at the tile's
// last step. Steps are the 64-key halves of every key tile in tile order, a
// tile's halves consecutive (an empty tile one step with no valid key, so
// every tile gets its statistic), through a 4-slot K ring.

constexpr int kStatThreads = 1024;
constexpr int kStatItems = 4;

template <int HEAT>
__global__ void __launch_bounds__(kStatThreads) tstats_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[4][kHalfBytes];
  __shared__ uint16_t steps[2 * kMaxBlocks];  // (key tile << 2) | (half << 1) | last of tile
  __shared__ uint8_t tvc[kMaxBlocks];
  __shared__ int32_t step_total;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int pick = wave >> 2, rg = wave & 3;
  const int li = lane & 31, hi = lane >> 5;
  const int64_t n_groups = (p.n_q_tiles + kStatItems - 1) / kStatItems;
  const int64_t head = blockIdx.x / n_groups;
  const int64_t r = (blockIdx.x % n_groups) * kStatItems + pick;
  const bool item_ok = r < p.n_q_tiles;
  const int64_t qrow = r * kTile + 32 * rg + li;  // row of lse / part
  const int64_t qtile = item_ok ? (p.q_tiles != nullptr ? p.q_tiles[r] : r) : -1;
  const bool qtile_ok = qtile >= 0 && qtile < p.q_tiles_held;
  const int64_t qsrc = (qtile_ok ? qtile : 0) * kTile + 32 * rg + li;
  const int nk = (int)p.n_k_tiles;

  for (int j = tid; j < nk; j += kStatThreads) tvc[j] = (uint8_t)min(max(p.valid_count[j], 0), kTile);
  if (wave == 0) {
    int n = 0;
    for (int j0 = 0; j0 < nk; j0 += 64) {
      const int j = j0 + lane;
      const bool one = j < nk;
      const bool two = one && p.valid_count[j] > kHalf;
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

  WaveState w;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const u32x4 v =
        qtile_ok ? ld16(p.q + qsrc * p.qs + head * p.qh + 16 * s + 8 * hi) : u32x4{0, 0, 0, 0};
    w.qf[s] = as_bf16x8(v);
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" : : "v"(w.qf[s]));
  w.m_run = -INFINITY;
  w.l_run = 0.f;
  w.mu = 0.f;
  w.blk = HEAT == kHeatMax ? -INFINITY : 0.f;
  __syncthreads();  // step list and valid counts ready
  const int n_steps = __builtin_amdgcn_readfirstlane(step_total);

  const float c = p.scale_log2;
  const HFrag fa = hfrag_offsets(0, lane), fb = hfrag_offsets(1, lane);
  // this wave's 1 KB K segment of a step: rows 4 wave + lane / 16, LDS chunk
  // lane % 16 holding logical chunk (lane % 16) ^ (row & 15); a segment
  // wholly past the valid count re-reads rows lane / 16
  uint32_t koff, kskip;
  {
    const int lr = lane >> 4, pc = lane & 15, row = 4 * wave + lr;
    const int kc = (pc ^ (row & 15)) << 3;
    koff = (uint32_t)((row * p.ks + kc) * 2);
    kskip = (uint32_t)((lr * p.ks + kc) * 2);
  }
  const uint16_t* kbase = p.k + head * p.kh;
  auto entry = [&](int u) { return __builtin_amdgcn_readfirstlane((int)steps[u]); };
  auto valid_of = [&](int e) {
    const int vc = __builtin_amdgcn_readfirstlane((int)tvc[e >> 2]);
    return (e & 2) ? vc - kHalf : min(vc, kHalf);
  };
  auto load_step = [&](int u, lds_u8* slot) {
    const int e = entry(u);
    const int64_t row0 = (int64_t)(e >> 2) * kTile + ((e >> 1) & 1) * kHalf;
    const char* b = reinterpret_cast<const char*>(kbase + row0 * p.ks);
    dma16(b, 4 * wave < valid_of(e) ? koff : kskip, slot + wave * 1024);
  };
  // One step over the step's vch valid keys (sub-block B only when vch > 32).
  // 'sum': once a row has a reference, the step's probabilities are taken
  // against it as it stands and kept unless their sum could lose range
  // (2^64 or more, or not finite), so most steps skip the row max; such a
  // step, a row's first one, and every 'max' step run the online softmax as
  // the sparse forward does (reference raised past a slack of 8).
  auto step = [&](const lds_u8* slot, int vch) {
    const f32x16 sa = sub_scores(slot, fa, w, vch, hi);
    f32x16 sb;
    const bool two = vch > 32;
    if (two) sb = sub_scores(slot, fb, w, vch - 32, hi);
    if (HEAT == kHeatSum && __all(w.m_run != -INFINITY)) {
      const float mu = w.mu;
      float l4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        l4[e >> 2] += __builtin_amdgcn_exp2f(fmaf(sa[e], c, -mu));
        if (two) l4[e >> 2] += __builtin_amdgcn_exp2f(fmaf(sb[e], c, -mu));
      }
      const float lsum = (l4[0] + l4[1]) + (l4[2] + l4[3]);
      if (__all(lsum < 0x1p64f)) {
        w.l_run += lsum;
        w.blk += lsum;
        return;
      }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, two ? fmaxf(sa[e], sb[e]) : sa[e]);
    const float mraw = half_swap_max(mloc);  // the row's raw max over the step's keys
    mloc = mraw * c;
    const float m_new = mloc > w.m_run + kRescaleSlack ? mloc : w.m_run;
    const float mu = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - mu);
    w.m_run = m_new;
    w.mu = mu;
    if (HEAT == kHeatMax) w.blk = fmaxf(w.blk, mraw);
    float l4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      l4[e >> 2] += __builtin_amdgcn_exp2f(fmaf(sa[e], c, -mu));
      if (two) l4[e >> 2] += __builtin_amdgcn_exp2f(fmaf(sb[e], c, -mu));
    }
    const float lsum = (l4[0] + l4[1]) + (l4[2] + l4[3]);
    w.l_run = fmaf(w.l_run, alpha, lsum);
    if (HEAT == kHeatSum) w.blk = fmaf(w.blk, alpha, lsum);
  };
  // At a tile's last step: its log2 statistic per row (log-sum-exp for
  // 'sum', the bf16-rounded raw max times the scale for 'max', as the
  // reference's heat rounds scores to bf16 before scaling).
  auto flush = [&](int j) {
    float l;
    if (HEAT == kHeatSum) {
      const float tot = half_swap_sum(w.blk);
      l = tot > 0.f ? __log2f(tot) + w.mu : -INFINITY;
      w.blk = 0.f;
    } else {
      l = bf16_to_f32(f32_to_bf16(w.blk)) * c;
      w.blk = -INFINITY;
    }
    if (item_ok && hi == 0) p.part[head * p.part_sh + (int64_t)j * p.part_st + qrow] = l;
  };
  auto compute_step = [&](int u, const lds_u8* slot) {
    const int e = entry(u);
    const int vch = valid_of(e);
    if (vch > 0) step(slot, vch);
    if (e & 1) flush(e >> 2);
  };
  lds_u8* K0 = (lds_u8*)ring[0];
  lds_u8* K1 = (lds_u8*)ring[1];
  lds_u8* K2 = (lds_u8*)ring[2];
  lds_u8* K3 = (lds_u8*)ring[3];
  // The ring: step u in slot u & 3; at the top of step u its own load is
  // waited for (those of u+1, u+2 may stay in flight), then a bare barrier,
  // then the slot step u-1 used is refilled with step u+3.
  auto top = [&](int u) {
    if (u + 2 < n_steps) VEDA_WAIT_VM(2);
    else if (u + 1 < n_steps) VEDA_WAIT_VM(1);
    else VEDA_WAIT_VM(0);
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
  const float l = half_swap_sum(w.l_run);
  if (item_ok && hi == 0)
    p.lse[head * p.lse_sh + qrow * p.lse_ss] = l > 0.f ? (w.m_run + __log2f(l)) * kLn2 : -INFINITY;
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
                                     int64_t lse_stride_h, int64_t lse_stride_s,
                                     int64_t front_tiles, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_sparse_fwd: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(front_tiles >= 0 && front_tiles <= n_q_tiles,
               "block_sparse_fwd: front_tiles %lld outside [0, n_q_tiles]", (long long)front_tiles);
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
  p.q_rows = n_q_tiles * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = lse; p.lse_sh = lse_stride_h; p.lse_ss = lse_stride_s;
  p.front = front_tiles;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  sfwd_kernel<kSparse><<<(unsigned)items, kThreads2, 0, s>>>(p);
  return check_launch("veda_block_sparse_fwd");
}

extern "C" int veda_block_sparse_fwd_seq(
    const void* q, int64_t q_rows, int64_t seq_heads, int64_t q_stride_s, int64_t q_stride_h,
    const int64_t* gather_index, const int64_t* scatter_index, const int32_t* slot_valid,
    const int64_t* heads, int64_t n_heads, const void* k, int64_t k_stride_s, int64_t k_stride_h,
    const void* v, int64_t v_stride_s, int64_t v_stride_h, int64_t head_dim, int64_t n_q_tiles,
    int64_t n_k_tiles, const int32_t* full_cnt, const int32_t* full_idx, const int32_t* part_cnt,
    const int32_t* part_idx, int64_t list_ld, const int32_t* valid_count, float scale, void* out,
    int64_t out_rows, int64_t o_stride_s, int64_t o_stride_h, int64_t front_tiles, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_sparse_fwd_seq: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(front_tiles >= 0 && front_tiles <= n_q_tiles,
               "block_sparse_fwd_seq: front_tiles %lld outside [0, n_q_tiles]",
               (long long)front_tiles);
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0 && n_k_tiles >= 0 && q_rows >= 0 && out_rows >= 0 &&
                   seq_heads >= 0,
               "block_sparse_fwd_seq: negative size");
  VEDA_REQUIRE(list_ld >= n_k_tiles, "block_sparse_fwd_seq: list_ld %lld < n_k_tiles %lld",
               (long long)list_ld, (long long)n_k_tiles);
  VEDA_REQUIRE(gather_index != nullptr && scatter_index != nullptr && slot_valid != nullptr &&
                   heads != nullptr,
               "block_sparse_fwd_seq: the gather / scatter indices, slot_valid and heads are required");
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                   q_stride_s % 8 == 0 && q_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   k_stride_h % 8 == 0 && v_stride_s % 8 == 0 && v_stride_h % 8 == 0 &&
                   o_stride_s % 4 == 0 && o_stride_h % 4 == 0,
               "block_sparse_fwd_seq: rows must be 16-byte aligned");
  const int64_t items = n_heads * n_q_tiles;
  if (items == 0) return VEDA_OK;
  VEDA_REQUIRE(n_k_tiles >= 1 && n_k_tiles <= kMaxBlocks,
               "block_sparse_fwd_seq: n_k_tiles %lld outside [1, %d]", (long long)n_k_tiles,
               kMaxBlocks);
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
  p.q_rows = n_q_tiles * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = nullptr;
  p.front = front_tiles;
  p.seq_q = gather_index;
  p.seq_o = scatter_index;
  p.slot_ok = slot_valid;
  p.seq_heads = heads;
  p.seq_rows = q_rows;
  p.seq_heads_n = seq_heads;
  p.out_rows = out_rows;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  sfwd_kernel<kSparse><<<(unsigned)items, kThreads2, 0, s>>>(p);
  return check_launch("veda_block_sparse_fwd_seq");
}

extern "C" int veda_block_sparse_fwd_seq_kv(
    const void* q, const void* k, const void* v, int64_t q_rows, int64_t seq_heads,
    int64_t stride_s, int64_t stride_h, const int64_t* gather_index, const int64_t* scatter_index,
    const int32_t* slot_valid, const int64_t* heads, int64_t n_heads, int64_t head_dim,
    int64_t n_q_tiles, int64_t n_k_tiles, const int32_t* full_cnt, const int32_t* full_idx,
    const int32_t* part_cnt, const int32_t* part_idx, int64_t list_ld, const int32_t* valid_count,
    float scale, void* out, int64_t out_rows, int64_t o_stride_s, int64_t o_stride_h,
    int64_t front_tiles, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "block_sparse_fwd_seq_kv: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(front_tiles >= 0 && front_tiles <= n_q_tiles,
               "block_sparse_fwd_seq_kv: front_tiles %lld outside [0, n_q_tiles]",
               (long long)front_tiles);
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0 && n_k_tiles >= 0 && q_rows >= 0 && out_rows >= 0 &&
                   seq_heads >= 0,
               "block_sparse_fwd_seq_kv: negative size");
  VEDA_REQUIRE(list_ld >= n_k_tiles, "block_sparse_fwd_seq_kv: list_ld %lld < n_k_tiles %lld",
               (long long)list_ld, (long long)n_k_tiles);
  VEDA_REQUIRE(gather_index != nullptr && scatter_index != nullptr && slot_valid != nullptr &&
                   heads != nullptr,
               "block_sparse_fwd_seq_kv: the gather / scatter indices, slot_valid and heads are "
               "required");
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                   stride_s % 8 == 0 && stride_h % 8 == 0 && o_stride_s % 4 == 0 &&
                   o_stride_h % 4 == 0,
               "block_sparse_fwd_seq_kv: rows must be 16-byte aligned");
  const int64_t items = n_heads * n_q_tiles;
  if (items == 0) return VEDA_OK;
  VEDA_REQUIRE(n_k_tiles >= 1 && n_k_tiles <= kMaxBlocks,
               "block_sparse_fwd_seq_kv: n_k_tiles %lld outside [1, %d]", (long long)n_k_tiles,
               kMaxBlocks);
  VEDA_REQUIRE(q_rows >= 1 && seq_heads >= 1, "block_sparse_fwd_seq_kv: k and v need rows and heads");
  // a key row's byte offset from its head's first row is a 32-bit load offset
  VEDA_REQUIRE(q_rows < ((int64_t)1 << 31) && (q_rows - 1) * stride_s * 2 + 2 * kD < (int64_t)1 << 32,
               "block_sparse_fwd_seq_kv: %lld rows of stride %lld exceed the 4 GiB load offset",
               (long long)q_rows, (long long)stride_s);
  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.qs = stride_s; p.qh = stride_h;
  p.ks = stride_s; p.kh = stride_h;
  p.vs = stride_s; p.vh = stride_h;
  p.n_heads = n_heads; p.n_q_tiles = n_q_tiles; p.n_k_tiles = n_k_tiles;
  p.full_cnt = full_cnt; p.full_idx = full_idx;
  p.part_cnt = part_cnt; p.part_idx = part_idx;
  p.list_ld = list_ld;
  p.valid_count = valid_count;
  p.q_rows = n_q_tiles * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = nullptr;
  p.front = front_tiles;
  p.seq_q = gather_index;
  p.seq_o = scatter_index;
  p.slot_ok = slot_valid;
  p.seq_heads = heads;
  p.seq_rows = q_rows;
  p.seq_heads_n = seq_heads;
  p.out_rows = out_rows;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  sfwd_kernel<kSparse, true><<<(unsigned)items, kThreads2, 0, s>>>(p);
  return check_launch("veda_block_sparse_fwd_seq_kv");
}

extern "C" int veda_compensated_attention(
    const void* q, int64_t q_stride_s, int64_t q_stride_h, const void* k, int64_t k_stride_s,
    int64_t k_stride_h, const void* v, int64_t v_stride_s, int64_t v_stride_h, int64_t n_heads,
    int64_t head_dim, int64_t n_q_tiles, int64_t n_k_tiles, const int32_t* full_cnt,
    const int32_t* full_idx, const int32_t* part_cnt, const int32_t* part_idx, int64_t list_ld,
    const void* kc, const void* vc, int64_t c_stride_s, int64_t c_stride_h, const uint8_t* keep,
    const int32_t* valid_count, float scale, void* out, int64_t o_stride_s, int64_t o_stride_h,
    int64_t front_tiles, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "compensated_attention: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(front_tiles >= 0 && front_tiles <= n_q_tiles,
               "compensated_attention: front_tiles %lld outside [0, n_q_tiles]",
               (long long)front_tiles);
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0 && n_k_tiles >= 0,
               "compensated_attention: negative size");
  VEDA_REQUIRE(list_ld >= n_k_tiles, "compensated_attention: list_ld %lld < n_k_tiles %lld",
               (long long)list_ld, (long long)n_k_tiles);
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(kc) && aligned16(vc) &&
                   aligned16(out) && q_stride_s % 8 == 0 && q_stride_h % 8 == 0 &&
                   k_stride_s % 8 == 0 && k_stride_h % 8 == 0 && v_stride_s % 8 == 0 &&
                   v_stride_h % 8 == 0 && c_stride_s % 8 == 0 && c_stride_h % 8 == 0 &&
                   o_stride_s % 4 == 0 && o_stride_h % 4 == 0,
               "compensated_attention: rows must be 16-byte aligned");
  VEDA_REQUIRE(2 * c_stride_s < (1 << 24), "compensated_attention: summary stride too large");
  const int64_t items = n_heads * n_q_tiles;
  if (items == 0) return VEDA_OK;
  VEDA_REQUIRE(n_k_tiles >= 1 && n_k_tiles <= kMaxBlocks,
               "compensated_attention: n_k_tiles %lld outside [1, %d]", (long long)n_k_tiles,
               kMaxBlocks);
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
  p.q_rows = n_q_tiles * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.keep = keep;
  p.kc = static_cast<const uint16_t*>(kc);
  p.vc = static_cast<const uint16_t*>(vc);
  p.cs = c_stride_s; p.ch = c_stride_h;
  p.front = front_tiles;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  sfwd_kernel<kSparseComp><<<(unsigned)items, kThreads2, 0, s>>>(p);
  return check_launch("veda_compensated_attention");
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
  p.q_rows = seq_len;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = lse; p.lse_sh = lse_stride_h; p.lse_ss = lse_stride_s;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  sfwd_kernel<kDenseRows><<<(unsigned)items, kThreads2, 0, s>>>(p);
  return check_launch("veda_dense_fwd");
}

extern "C" int veda_dense_heat_fwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                                   int64_t q_tiles_held, const void* k, int64_t k_stride_s,
                                   int64_t k_stride_h, const void* v, int64_t v_stride_s,
                                   int64_t v_stride_h, int64_t n_heads, int64_t head_dim,
                                   const int64_t* q_tiles, int64_t n_items, int64_t n_k_tiles,
                                   const int32_t* valid_count, float scale, int reduce,
                                   void* out, int64_t o_stride_s, int64_t o_stride_h, float* lse,
                                   int64_t lse_stride_h, int64_t lse_stride_s, float* part,
                                   void* stream) {
  VEDA_REQUIRE(head_dim == kD, "dense_heat_fwd: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(reduce == 0 || reduce == 1, "dense_heat_fwd: reduce must be 0 (sum) or 1 (max)");
  VEDA_REQUIRE(n_heads >= 0 && n_items >= 0 && q_tiles_held >= 0,
               "dense_heat_fwd: negative size");
  VEDA_REQUIRE(q_tiles != nullptr || n_items <= q_tiles_held,
               "dense_heat_fwd: %lld items but q holds %lld tiles", (long long)n_items,
               (long long)q_tiles_held);
  VEDA_REQUIRE(lse != nullptr && part != nullptr, "dense_heat_fwd: lse and part are required");
  VEDA_REQUIRE((out == nullptr) == (v == nullptr),
               "dense_heat_fwd: out and v go together (out needs P.V)");
  VEDA_REQUIRE(aligned16(q) && aligned16(k) && (v == nullptr || aligned16(v)) &&
                   (out == nullptr || aligned16(out)) && q_stride_s % 8 == 0 &&
                   q_stride_h % 8 == 0 && k_stride_s % 8 == 0 && k_stride_h % 8 == 0 &&
                   (v == nullptr || (v_stride_s % 8 == 0 && v_stride_h % 8 == 0)) &&
                   (out == nullptr || (o_stride_s % 4 == 0 && o_stride_h % 4 == 0)),
               "dense_heat_fwd: rows must be 16-byte aligned");
  const int64_t items = n_heads * n_items;
  if (items == 0) return VEDA_OK;
  VEDA_REQUIRE(n_k_tiles >= 1 && n_k_tiles <= kMaxBlocks,
               "dense_heat_fwd: n_k_tiles %lld outside [1, %d]", (long long)n_k_tiles, kMaxBlocks);
  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = v != nullptr ? static_cast<const uint16_t*>(v) : p.k;
  p.qs = q_stride_s; p.qh = q_stride_h;
  p.ks = k_stride_s; p.kh = k_stride_h;
  p.vs = v != nullptr ? v_stride_s : k_stride_s;
  p.vh = v != nullptr ? v_stride_h : k_stride_h;
  p.n_heads = n_heads; p.n_q_tiles = n_items; p.n_k_tiles = n_k_tiles;
  p.valid_count = valid_count;
  p.used = 0;
  p.q_rows = n_items * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.lse = lse; p.lse_sh = lse_stride_h; p.lse_ss = lse_stride_s;
  p.q_tiles = q_tiles;
  p.q_tiles_held = q_tiles_held;
  p.part = part;
  p.part_st = n_items * kTile;
  p.part_sh = n_k_tiles * p.part_st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned g = (unsigned)items;
  if (out != nullptr) {
    if (reduce) hfwd_kernel<kHeatMax><<<g, kThreads, 0, s>>>(p);
    else hfwd_kernel<kHeatSum><<<g, kThreads, 0, s>>>(p);
  } else {
    const unsigned gs = (unsigned)(n_heads * ((n_items + kStatItems - 1) / kStatItems));
    if (reduce) tstats_kernel<kHeatMax><<<gs, kStatThreads, 0, s>>>(p);
    else tstats_kernel<kHeatSum><<<gs, kStatThreads, 0, s>>>(p);
  }
  return check_launch("veda_dense_heat_fwd");
}

extern "C" int veda_zero_order_compensation(
    const void* o_kept, int64_t ok_stride_s, int64_t ok_stride_h, const float* lse_kept,
    int64_t lse_stride_h, int64_t lse_stride_s, const void* q, int64_t q_stride_s,
    int64_t q_stride_h, const void* kc, const void* vc, int64_t c_stride_s, int64_t c_stride_h,
    const uint8_t* keep, const int32_t* valid_count, int64_t n_heads, int64_t head_dim,
    int64_t n_q_tiles, int64_t n_k_tiles, float scale, void* out, int64_t o_stride_s,
    int64_t o_stride_h, void* stream) {
  VEDA_REQUIRE(head_dim == kD, "zero_order_compensation: head_dim must be 128, got %lld",
               (long long)head_dim);
  VEDA_REQUIRE(n_heads >= 0 && n_q_tiles >= 0, "zero_order_compensation: negative size");
  VEDA_REQUIRE(aligned16(q) && aligned16(kc) && aligned16(vc) && aligned16(out) &&
                   (reinterpret_cast<uintptr_t>(o_kept) & 7u) == 0 && q_stride_s % 8 == 0 &&
                   q_stride_h % 8 == 0 && c_stride_s % 8 == 0 && c_stride_h % 8 == 0 &&
                   o_stride_s % 4 == 0 && o_stride_h % 4 == 0 && ok_stride_s % 4 == 0 &&
                   ok_stride_h % 4 == 0,
               "zero_order_compensation: rows must be aligned");
  VEDA_REQUIRE(2 * c_stride_s < (1 << 24), "zero_order_compensation: summary stride too large");
  const int64_t items = n_heads * n_q_tiles;
  if (items == 0) return VEDA_OK;
  VEDA_REQUIRE(n_k_tiles >= 1 && n_k_tiles <= kMaxBlocks,
               "zero_order_compensation: n_k_tiles %lld outside [1, %d]", (long long)n_k_tiles,
               kMaxBlocks);
  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.kc = static_cast<const uint16_t*>(kc);
  p.vc = static_cast<const uint16_t*>(vc);
  p.cs = c_stride_s; p.ch = c_stride_h;
  p.qs = q_stride_s; p.qh = q_stride_h;
  p.n_heads = n_heads; p.n_q_tiles = n_q_tiles; p.n_k_tiles = n_k_tiles;
  p.valid_count = valid_count;
  p.q_rows = n_q_tiles * kTile;
  p.scale_log2 = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.os = o_stride_s; p.oh = o_stride_h;
  p.keep = keep;
  p.o_kept = static_cast<const uint16_t*>(o_kept);
  p.oks = ok_stride_s; p.okh = ok_stride_h;
  p.lse_kept = lse_kept; p.lk_h = lse_stride_h; p.lk_s = lse_stride_s;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  sfwd_kernel<kVirtualOnly><<<(unsigned)items, kThreads2, 0, s>>>(p);
  return check_launch("veda_zero_order_compensation");
}
