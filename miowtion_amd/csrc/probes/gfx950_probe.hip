// Micro-probes of the gfx950 properties the attention kernels are laid out
// for (not part of the library; built by the Makefile beside this file).
//
//   gfx950_probe rates   LDS read rates, VALU instruction costs, MFMA/VALU
//                        overlap across two waves of a SIMD and inside one
//   gfx950_probe lanes   512 single-wave dispatches for the LDS lane-group
//                        study (run under rocprofv3 by lds_lanes.py)
//   gfx950_probe dma     global -> LDS load rate per CU from an L2-resident
//                        buffer: global_load_lds_dwordx4 against plain
//                        global_load_dwordx4 (and with a ds_write_b128)
//
// Every access stays inside the kernel's own LDS array or its output
// buffer; every loop has a fixed trip count.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));             \
      return 1;                                                           \
    }                                                                     \
  } while (0)

// ---------------------------------------------------------------------------
// LDS read rate: one workgroup of 8 waves per CU, batches of 8 reads (inline
// asm, then one wait), every address inside a 64 KB array.
//   0: ds_read_b128, each lane its own 16 bytes of a 1 KB row block
//   1: ds_read_b64, linear
//   2: ds_read_b64_tr_b16, linear
//   3: ds_read_b64_tr_b16 in the backward's 16-key fragment pattern with the
//      32-row chunk swizzle ((r % 4) << 2 | (r / 4) % 4)
//   4: the same pattern with the 16-row swizzle ((r % 4) << 2 | ((r / 4) % 2) << 1 | (r / 8) % 2)
//   5: ds_read_b128 of 16-key rows with the 16-row swizzle
//   6: ds_read_b128 of 32-row fragments with the 32-row swizzle
constexpr int kBatches = 1024;

__device__ __forceinline__ int swz32(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int swz16(int r) {
  return ((r & 3) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
}

#define LDS_RD(OP, V, A, OFF) asm volatile(OP " %0, %1 offset:" #OFF : "=v"(V) : "v"(A))
#define LDS_BATCH(OP, T)                                                                  \
  {                                                                                       \
    T v0, v1, v2, v3, v4, v5, v6, v7;                                                     \
    LDS_RD(OP, v0, a, 0);                                                                 \
    LDS_RD(OP, v1, a, 4096);                                                              \
    LDS_RD(OP, v2, a, 8192);                                                              \
    LDS_RD(OP, v3, a, 12288);                                                             \
    LDS_RD(OP, v4, a, 16384);                                                             \
    LDS_RD(OP, v5, a, 20480);                                                             \
    LDS_RD(OP, v6, a, 24576);                                                             \
    LDS_RD(OP, v7, a, 28672);                                                             \
    asm volatile("s_waitcnt lgkmcnt(0)" ::"v"(v0), "v"(v1), "v"(v2), "v"(v3), "v"(v4),    \
                 "v"(v5), "v"(v6), "v"(v7));                                              \
  }

template <int MODE>
__global__ void __launch_bounds__(512) lds_rate_kernel(uint32_t* out) {
  __shared__ __attribute__((aligned(16))) uint8_t buf[65536];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < 65536 / 4; i += 512) reinterpret_cast<uint32_t*>(buf)[i] = i * 2654435761u;
  __syncthreads();
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)buf;
  const int n = lane & 15, g = lane >> 4, rr = 4 * g + (n >> 2);
  uint32_t a0;
  if (MODE == 0) a0 = (wave * 4096 + lane * 16) & 32767;
  else if (MODE == 1 || MODE == 2) a0 = (wave * 2048 + lane * 8) & 32767;
  else if (MODE == 3) a0 = rr * 256 + ((((n >> 1) & 1) ^ swz32(rr)) << 4) + 8 * (n & 1) + (wave & 3) * 4096;
  else if (MODE == 4) a0 = rr * 256 + ((((n >> 1) & 1) ^ swz16(rr)) << 4) + 8 * (n & 1) + (wave & 3) * 4096;
  else if (MODE == 5) a0 = n * 256 + ((g ^ swz16(n)) << 4) + (wave & 3) * 4096;
  else {
    const int li = lane & 31, hi = lane >> 5;
    a0 = li * 256 + ((hi ^ swz32(li)) << 4) + (wave & 1) * 8192;
  }
  for (int it = 0; it < kBatches; ++it) {
    const uint32_t a = base + (a0 ^ ((it & 7) << 5));  // stays inside the same 256-byte row
    if (MODE == 0 || MODE >= 5) LDS_BATCH("ds_read_b128", u32x4)
    else if (MODE == 1) LDS_BATCH("ds_read_b64", u32x2)
    else LDS_BATCH("ds_read_b64_tr_b16", u32x2)
  }
  out[blockIdx.x * 512 + tid] = a0;
}

// ---------------------------------------------------------------------------
// VALU cost per wave64 instruction and SIMD: 256 workgroups of 8 waves (two
// per SIMD), eight independent chains per lane, inline asm so the compiler
// neither folds nor reorders the instruction under test.
constexpr int kValuIters = 4096;
#define CH1(I)                                                                               \
  asm volatile(I " %0, %0\n\t" I " %1, %1\n\t" I " %2, %2\n\t" I " %3, %3\n\t" I " %4, %4\n\t" \
               I " %5, %5\n\t" I " %6, %6\n\t" I " %7, %7"                                       \
               : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7))
#define CH2(I)                                                                                \
  asm volatile(I " %0, %0, %8\n\t" I " %1, %1, %8\n\t" I " %2, %2, %8\n\t" I " %3, %3, %8\n\t"   \
               I " %4, %4, %8\n\t" I " %5, %5, %8\n\t" I " %6, %6, %8\n\t" I " %7, %7, %8"      \
               : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7) \
               : "v"(y))
#define CH3(I)                                                                                  \
  asm volatile(I " %0, %0, %8, %0\n\t" I " %1, %1, %8, %1\n\t" I " %2, %2, %8, %2\n\t"             \
               I " %3, %3, %8, %3\n\t" I " %4, %4, %8, %4\n\t" I " %5, %5, %8, %5\n\t"            \
               I " %6, %6, %8, %6\n\t" I " %7, %7, %8, %7"                                       \
               : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7) \
               : "v"(y))

template <int OP>
__global__ void __launch_bounds__(512) valu_kernel(float* out) {
  float x0 = 0.5f + threadIdx.x, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5,
        x6 = x0 + 6, x7 = x0 + 7;
  const float y = 0.999f;
  for (int it = 0; it < kValuIters; ++it) {
    if (OP == 0) CH2("v_add_f32");
    else if (OP == 1) CH3("v_fma_f32");
    else if (OP == 2) CH2("v_max_f32");
    else if (OP == 3) CH3("v_max3_f32");
    else if (OP == 4) CH2("v_cvt_pk_bf16_f32");
    else if (OP == 5) CH1("v_exp_f32");
    else if (OP == 6) CH1("v_exp_f16");
    else CH1("v_rcp_f32");
  }
  out[blockIdx.x * 512 + threadIdx.x] = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7;
}

// ---------------------------------------------------------------------------
// MFMA / VALU overlap. An iteration is 8 independent 32x32x16 bf16 MFMAs
// (accumulators c0..c7) and/or VREP VALU blocks (per chain: v_exp_f32, two
// v_fma_f32, v_max_f32; 8 chains), each as one asm block.
//   ROLE 0: MFMA only   1: VALU only   2: both, interleaved in one wave
//   (after each MFMA one chain's 4 VREP VALU instructions)
// Workgroups carry 96 KB of dynamic LDS so that one fits a CU; 256 threads
// give one wave per SIMD, 512 two.
constexpr int kOverlapIters = 2048;
#define MF(C) "v_mfma_f32_32x32x16_bf16 " C ", %[a], %[b], " C "\n\t"
#define VB(X)                                                                                   \
  "v_exp_f32 " X ", " X "\n\tv_fma_f32 " X ", " X ", %[y], " X "\n\tv_fma_f32 " X ", " X ", %[y], " X \
  "\n\tv_max_f32 " X ", " X ", %[y]\n\t"
#define ACC_OUT                                                                                  \
  [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [c3] "+v"(c3), [c4] "+v"(c4), [c5] "+v"(c5),      \
      [c6] "+v"(c6), [c7] "+v"(c7)
#define X_OUT                                                                                    \
  [x0] "+v"(x0), [x1] "+v"(x1), [x2] "+v"(x2), [x3] "+v"(x3), [x4] "+v"(x4), [x5] "+v"(x5),      \
      [x6] "+v"(x6), [x7] "+v"(x7)

template <int ROLE, int VREP>
__device__ __forceinline__ void overlap_body(float* out) {
  const int tid = threadIdx.x;
  f32x16 c0, c1, c2, c3, c4, c5, c6, c7;
  for (int e = 0; e < 16; ++e) c0[e] = c1[e] = c2[e] = c3[e] = c4[e] = c5[e] = c6[e] = c7[e] = 0.f;
  const u32x4 a = {0x3c003c00u + (uint32_t)tid, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u}, b = a;
  float x0 = 0.1f * tid, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5, x6 = x0 + 6,
        x7 = x0 + 7;
  const float y = 0.999f;
  for (int it = 0; it < kOverlapIters; ++it) {
    if (ROLE == 0) {
      asm volatile(MF("%[c0]") MF("%[c1]") MF("%[c2]") MF("%[c3]") MF("%[c4]") MF("%[c5]") MF("%[c6]")
                       MF("%[c7]")
                   : ACC_OUT
                   : [a] "v"(a), [b] "v"(b));
    } else if (ROLE == 1) {
#pragma unroll
      for (int r = 0; r < VREP; ++r)
        asm volatile(VB("%[x0]") VB("%[x1]") VB("%[x2]") VB("%[x3]") VB("%[x4]") VB("%[x5]")
                         VB("%[x6]") VB("%[x7]")
                     : X_OUT
                     : [y] "v"(y));
    } else if (VREP == 1) {
      asm volatile(MF("%[c0]") VB("%[x0]") MF("%[c1]") VB("%[x1]") MF("%[c2]") VB("%[x2]") MF("%[c3]")
                       VB("%[x3]") MF("%[c4]") VB("%[x4]") MF("%[c5]") VB("%[x5]") MF("%[c6]")
                           VB("%[x6]") MF("%[c7]") VB("%[x7]")
                   : ACC_OUT, X_OUT
                   : [a] "v"(a), [b] "v"(b), [y] "v"(y));
    } else {
      asm volatile(MF("%[c0]") VB("%[x0]") VB("%[x1]") MF("%[c1]") VB("%[x2]") VB("%[x3]")
                       MF("%[c2]") VB("%[x4]") VB("%[x5]") MF("%[c3]") VB("%[x6]") VB("%[x7]")
                           MF("%[c4]") VB("%[x0]") VB("%[x1]") MF("%[c5]") VB("%[x2]") VB("%[x3]")
                               MF("%[c6]") VB("%[x4]") VB("%[x5]") MF("%[c7]") VB("%[x6]") VB("%[x7]")
                   : ACC_OUT, X_OUT
                   : [a] "v"(a), [b] "v"(b), [y] "v"(y));
    }
  }
  // wait states before VALU reads of the last MFMA results
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float s = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7;
  for (int e = 0; e < 16; e += 5) s += c0[e] + c1[e] + c2[e] + c3[e] + c4[e] + c5[e] + c6[e] + c7[e];
  out[blockIdx.x * 512 + tid] = s;
}

// MODE 0..2: every wave takes role MODE; MODE 3: waves 0..3 (one per SIMD)
// MFMA only, waves 4..7 VALU only
template <int MODE, int VREP>
__global__ void __launch_bounds__(512) overlap_kernel(float* out) {
  extern __shared__ uint8_t pad[];
  if (MODE < 3) {
    overlap_body<MODE < 3 ? MODE : 0, VREP>(out);
  } else if (threadIdx.x < 256) {
    overlap_body<0, VREP>(out);
  } else {
    overlap_body<1, VREP>(out);
  }
  if (threadIdx.x == 0) pad[0] = 0;
}

// ---------------------------------------------------------------------------
// LDS lane groups: one wave, lanes a and b active, reading the same bank at
// different addresses (rows 0 and 1 of 256-byte rows, same column) 64 times;
// SQ_LDS_BANK_CONFLICT of the dispatch is non-zero iff a and b are served in
// the same cycle. Dispatch order: mode (b128, b64), a in {0, 5, 17, 42}, b in
// 0..63.
template <int MODE>
__global__ void __launch_bounds__(64) lane_kernel(uint32_t* out, int a, int b) {
  __shared__ __attribute__((aligned(16))) uint8_t buf[1024];
  const int lane = threadIdx.x;
  for (int i = lane; i < 256; i += 64) reinterpret_cast<uint32_t*>(buf)[i] = i;
  __syncthreads();
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)buf;
  uint32_t acc = 0;
  if (lane == a || lane == b) {
    const uint32_t addr = base + (lane == a ? 0u : 256u);
    for (int it = 0; it < 64; ++it) {
      if (MODE == 0) {
        u32x4 v;
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
        acc ^= v[0];
      } else {
        u32x2 v;
        asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
        acc ^= v[0];
      }
    }
  }
  out[lane] = acc;
}

constexpr int kLaneA[4] = {0, 5, 17, 42};

// ---------------------------------------------------------------------------
// Load rate into a CU: WAVES waves per workgroup, one workgroup per CU (64 KB
// of LDS), each wave kDmaBatches batches of 8 loads of 1 KB (64 lanes x 16 B)
// from a 1 MB buffer (L2-resident after the first pass), then a wait for
// all of them, as the sparse forward waits per step.
//   0: global_load_lds_dwordx4 into the wave's 8 KB of LDS
//   1: global_load_dwordx4 into registers
//   2: global_load_dwordx4 into registers, then ds_write_b128 of each
constexpr int kDmaBatches = 512;
constexpr uint32_t kDmaBufBytes = 1u << 20;

template <int MODE, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) dma_kernel(const char* src, uint32_t* out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[WAVES * 8192];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds + wave * 8192;
  uint32_t acc = 0;
  for (int it = 0; it < kDmaBatches; ++it) {
    // the wave's 8 KB window of the buffer moves by 8 KB per batch
    const uint32_t win = ((blockIdx.x * WAVES + wave) * 8192u + it * 8192u) & (kDmaBufBytes - 1);
    const uint32_t voff = win + lane * 16;
    if (MODE == 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t m0 = lds_base + k * 1024;
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                     :
                     : "v"(voff + k * 1024), "s"(src), "s"(m0)
                     : "memory", "m0");
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      u32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v[k]) : "v"(voff + k * 1024), "s"(src));
      asm volatile("s_waitcnt vmcnt(0)" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]),
                   "v"(v[5]), "v"(v[6]), "v"(v[7]));
      if (MODE == 2) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          asm volatile("ds_write_b128 %0, %1" : : "v"(lds_base + k * 1024 + lane * 16), "v"(v[k]) : "memory");
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= v[k][0];
      }
    }
  }
  __syncthreads();
  out[blockIdx.x * 64 * WAVES + tid] = acc + lds[tid];
}

template <typename F>
static float time_ms(F launch) {
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  launch();  // warm-up
  (void)hipEventRecord(e0, 0);
  launch();
  (void)hipEventRecord(e1, 0);
  (void)hipEventSynchronize(e1);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return ms;
}

static int rates() {
  void* buf;
  CHECK(hipMalloc(&buf, 512 * 512 * 4));
  uint32_t* u = (uint32_t*)buf;
  float* f = (float*)buf;
  const char* lds_names[7] = {"ds_read_b128 (1 KB per instruction), linear",
                              "ds_read_b64 (512 B), linear",
                              "ds_read_b64_tr_b16 (512 B), linear",
                              "ds_read_b64_tr_b16, 16-key pattern, 32-row swizzle",
                              "ds_read_b64_tr_b16, 16-key pattern, 16-row swizzle",
                              "ds_read_b128, 16-key rows, 16-row swizzle",
                              "ds_read_b128, 32-row fragments, 32-row swizzle"};
  printf("LDS reads, 256 workgroups x 8 waves, %d batches of 8 per wave:\n", kBatches);
  for (int m = 0; m < 7; ++m) {
    float ms = time_ms([&] {
      switch (m) {
        case 0: lds_rate_kernel<0><<<256, 512>>>(u); break;
        case 1: lds_rate_kernel<1><<<256, 512>>>(u); break;
        case 2: lds_rate_kernel<2><<<256, 512>>>(u); break;
        case 3: lds_rate_kernel<3><<<256, 512>>>(u); break;
        case 4: lds_rate_kernel<4><<<256, 512>>>(u); break;
        case 5: lds_rate_kernel<5><<<256, 512>>>(u); break;
        default: lds_rate_kernel<6><<<256, 512>>>(u); break;
      }
    });
    CHECK(hipGetLastError());
    const double per_cu = 8.0 * kBatches * 8;  // wave-instructions per CU
    const double bytes = (m == 0 || m >= 5 ? 1024.0 : 512.0) * per_cu;
    printf("  %-52s %.3f ms: %.2f ns per instruction per CU, %.0f B/ns per CU\n", lds_names[m], ms,
           ms * 1e6 / per_cu, bytes / (ms * 1e6));
  }
  const char* valu_names[8] = {"v_add_f32", "v_fma_f32", "v_max_f32", "v_max3_f32",
                               "v_cvt_pk_bf16_f32", "v_exp_f32", "v_exp_f16", "v_rcp_f32"};
  printf("VALU, 256 workgroups x 8 waves (2 per SIMD), 8 chains x %d iterations:\n", kValuIters);
  for (int op = 0; op < 8; ++op) {
    float ms = time_ms([&] {
      switch (op) {
        case 0: valu_kernel<0><<<256, 512>>>(f); break;
        case 1: valu_kernel<1><<<256, 512>>>(f); break;
        case 2: valu_kernel<2><<<256, 512>>>(f); break;
        case 3: valu_kernel<3><<<256, 512>>>(f); break;
        case 4: valu_kernel<4><<<256, 512>>>(f); break;
        case 5: valu_kernel<5><<<256, 512>>>(f); break;
        case 6: valu_kernel<6><<<256, 512>>>(f); break;
        default: valu_kernel<7><<<256, 512>>>(f); break;
      }
    });
    CHECK(hipGetLastError());
    const double per_simd = 2.0 * kValuIters * 8;
    printf("  %-20s %.3f ms: %.2f ns per wave64 instruction per SIMD\n", valu_names[op], ms,
           ms * 1e6 / per_simd);
  }
  const size_t lds = 96 * 1024;
  const void* ov_kernels[2][4] = {
      {(const void*)overlap_kernel<0, 1>, (const void*)overlap_kernel<1, 1>,
       (const void*)overlap_kernel<2, 1>, (const void*)overlap_kernel<3, 1>},
      {(const void*)overlap_kernel<0, 2>, (const void*)overlap_kernel<1, 2>,
       (const void*)overlap_kernel<2, 2>, (const void*)overlap_kernel<3, 2>}};
  for (auto& row : ov_kernels)
    for (const void* k : row)
      CHECK(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  printf("MFMA / VALU overlap, 256 workgroups, %d iterations of 8 MFMAs and/or 32 x VREP VALU:\n",
         kOverlapIters);
  const char* ov_names[4] = {"MFMA only", "VALU only", "MFMA and VALU interleaved in each wave",
                             "one MFMA-only and one VALU-only wave per SIMD"};
  for (int vrep : {1, 2})
    for (int threads : {256, 512})
      for (int mode = 0; mode < 4; ++mode) {
        if ((mode == 3 && threads == 256) || (mode == 0 && vrep == 2)) continue;
        float ms = time_ms([&] {
          void* args[] = {&f};
          (void)hipLaunchKernel(ov_kernels[vrep - 1][mode], dim3(256), dim3(threads), args, lds, 0);
        });
        CHECK(hipGetLastError());
        printf("  VREP %d, %d wave(s) per SIMD, %-46s %.3f ms\n", vrep, threads / 256,
               ov_names[mode], ms);
      }
  CHECK(hipDeviceSynchronize());
  CHECK(hipFree(buf));
  return 0;
}

static int dma() {
  char* src;
  uint32_t* out;
  CHECK(hipMalloc(&src, kDmaBufBytes));
  CHECK(hipMemset(src, 1, kDmaBufBytes));
  CHECK(hipMalloc(&out, 256 * 512 * 4));
  const char* names[3] = {"global_load_lds_dwordx4 (to LDS)", "global_load_dwordx4 (to VGPRs)",
                          "global_load_dwordx4 + ds_write_b128"};
  printf("Loads into a CU, 256 workgroups (one per CU), %d batches of 8 x 1 KB per wave, "
         "1 MB L2-resident source:\n", kDmaBatches);
  for (int waves : {4, 8})
    for (int mode = 0; mode < 3; ++mode) {
      float ms = time_ms([&] {
        if (waves == 4) {
          if (mode == 0) dma_kernel<0, 4><<<256, 256>>>(src, out);
          else if (mode == 1) dma_kernel<1, 4><<<256, 256>>>(src, out);
          else dma_kernel<2, 4><<<256, 256>>>(src, out);
        } else {
          if (mode == 0) dma_kernel<0, 8><<<256, 512>>>(src, out);
          else if (mode == 1) dma_kernel<1, 8><<<256, 512>>>(src, out);
          else dma_kernel<2, 8><<<256, 512>>>(src, out);
        }
      });
      CHECK(hipGetLastError());
      const double bytes_cu = (double)waves * kDmaBatches * 8 * 1024;
      printf("  %d waves per CU, %-38s %.3f ms: %.0f B/ns per CU, %.1f TB/s total\n", waves,
             names[mode], ms, bytes_cu / (ms * 1e6), 256 * bytes_cu / (ms * 1e9));
    }
  CHECK(hipDeviceSynchronize());
  CHECK(hipFree(src));
  CHECK(hipFree(out));
  return 0;
}

static int lanes() {
  uint32_t* out;
  CHECK(hipMalloc(&out, 256));
  for (int mode = 0; mode < 2; ++mode)
    for (int ai = 0; ai < 4; ++ai)
      for (int b = 0; b < 64; ++b) {
        if (mode == 0) lane_kernel<0><<<1, 64>>>(out, kLaneA[ai], b);
        else lane_kernel<1><<<1, 64>>>(out, kLaneA[ai], b);
        CHECK(hipGetLastError());
      }
  CHECK(hipDeviceSynchronize());
  CHECK(hipFree(out));
  printf("lanes: 512 dispatches\n");
  return 0;
}

int main(int argc, char** argv) {
  if (argc == 2 && !strcmp(argv[1], "rates")) return rates();
  if (argc == 2 && !strcmp(argv[1], "lanes")) return lanes();
  if (argc == 2 && !strcmp(argv[1], "dma")) return dma();
  fprintf(stderr, "usage: %s rates|lanes|dma\n", argv[0]);
  return 2;
}
