// Building blocks shared by the pipelined MFMA kernels (attention and
// block heat): LDS pointer types, the HBM -> LDS load, wait counts, lane
// swaps and wave reductions.
#pragma once

#include "veda_common.h"

namespace veda {

constexpr int kHalf = 64;                       // keys per pipeline step
constexpr int kHalfBytes = kHalf * 128 * 2;     // 16 KB: K or V of a step (D = 128)

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

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

// Sum / max over all 64 lanes of a wave; every lane receives the result.
// Within a 16-lane row: DPP exchanges with lane ^ 1, lane ^ 2, the mirror
// inside 8 and the mirror inside 16 (each leaves the partial of a larger
// group in every lane); across rows: a swizzle with lane ^ 16, then the
// lane 32 positions away.
template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  auto dpp = [](float x, int ctrl) {
    switch (ctrl) {
      case 0: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0xB1, 0xF, 0xF, false));
      case 1: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x4E, 0xF, 0xF, false));
      case 2: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x141, 0xF, 0xF, false));
      default: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x140, 0xF, 0xF, false));
    }
  };
  v = op(v, dpp(v, 0));  // quad_perm [1, 0, 3, 2]: lane ^ 1
  v = op(v, dpp(v, 1));  // quad_perm [2, 3, 0, 1]: lane ^ 2
  v = op(v, dpp(v, 2));  // row_half_mirror: lane i <-> 7 - i inside 8
  v = op(v, dpp(v, 3));  // row_mirror: lane i <-> 15 - i inside 16
  // ds_swizzle bit mode (and 0x1f, or 0, xor 0x10): lane ^ 16 inside 32
  v = op(v, __uint_as_float(__builtin_amdgcn_ds_swizzle(__float_as_uint(v), 0x401F)));
  return MAX ? half_swap_max(v) : half_swap_sum(v);
}

// One 16-byte-per-lane HBM -> LDS load (global_load_lds_dwordx4): lane l
// reads 16 bytes at base + voff and writes them to LDS at dst + 16 l. It is
// issued as inline assembly so that the compiler's wait-count tracking does
// not see an LDS store behind it: that tracking merges conservatively at the
// loop head and would make the first fragment read of a step wait for every
// load in flight. The pipeline's explicit vmcnt waits order these loads;
// untracked loads only ever make the compiler's own vmcnt waits stricter.
// M0 (the LDS destination) is written inside the same statement, right
// before its use; nothing else in these kernels uses M0 (the compiler
// reports m0 as reserved in the clobber list and may not preserve it, which
// is why no value in it may live across the statement). The destination is
// wave-uniform by construction; readfirstlane states that to the compiler,
// which otherwise may keep it in a vector register after a per-lane select.
__device__ __forceinline__ void dma16(const char* base, uint32_t voff, const lds_u8* dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "s"(m0)
      : "memory", "m0");
}

// dma16 with the LDS destination given as its wave-uniform 32-bit LDS
// address (the value M0 takes), e.g. a per-wave slot base in a scalar
// register plus a constant segment offset.
__device__ __forceinline__ void dma16_m0(const char* base, uint32_t voff, uint32_t m0) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "s"(m0)
      : "memory", "m0");
}

// Workgroup order with the last `front` tiles of every head first: block b
// < heads * front takes (head b / front, tile n - front + b % front), the
// other blocks the remaining tiles head by head. Tiles that a mask makes
// dense (global rows or columns) have the longest walks; dispatching them
// first keeps them off the end of the launch. front = 0 is the plain
// (head, tile) order.
__device__ __forceinline__ void front_first(int64_t b, int64_t n_heads, int64_t n, int64_t front,
                                            int64_t& head, int64_t& tile) {
  const int64_t lead = n_heads * front;
  if (b < lead) {
    head = b / front;
    tile = n - front + b % front;
  } else {
    const int64_t rest = n - front;
    b -= lead;
    head = b / rest;
    tile = b % rest;
  }
}

// A hook called between the fragment reads and the products of a step (the
// walks issue the next step's loads there); the default does nothing.
struct NoHook {
  __device__ __forceinline__ void operator()(int) const {}
};

// vmcnt waits as s_waitcnt immediates (gfx9 encoding: vmcnt low bits [3:0],
// expcnt [6:4] and lgkmcnt [11:8] left at their maxima).
#define VEDA_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x0F70 | (n))

}  // namespace veda
