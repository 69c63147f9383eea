// MI355X characterisation probes behind hardware facts the kernel designs
// rely on.  Built into libmxprobes.so (not the kernel library) and driven by
// microbench/run.py; nothing in the kernel library calls them.
//
//  * mxp_overlap_launch: one workgroup of 4 waves per CU (150 KB of dynamic
//    LDS keeps a second one off), i.e. one wave per SIMD.  Every iteration
//    issues 8 independent 32x32x16 bf16 MFMAs, each followed in the same
//    scheduling region by a fixed mix of other instructions on independent
//    registers (32 VALU instructions of one kind per iteration, one s_nop
//    per MFMA, or both); with with_mfma = 0 the mix runs alone.  Lane 0 of each
//    workgroup writes the shader-clock cycles its loop took.  Comparing the
//    three timings (MFMAs alone, mix alone, both) shows how much of the mix
//    runs beside the wave's own MFMAs.
//  * mxp_mfma_rate_launch: the MFMA throughput of the whole chip, two waves
//    per SIMD (8-wave workgroups, one per CU), as 32x32x16 or 16x16x32 bf16
//    or 32x32x64 or 16x16x128 fp8 MFMAs on operands read from a caller
//    buffer: each wave rotates through
//    four A and four B fragments, so with random data the operands change
//    from one MFMA to the next, and with constant data they never do.  The
//    MFMA datapath's power, and with it the clock the chip holds, depends
//    on that.
//  * mxp_contend_launch: how a co-resident wave's work slows a wave's
//    MFMAs.  One 8-wave workgroup per CU: waves 0-3 issue 8 independent
//    MFMAs per iteration (bf16 32x32x16 or fp8 32x32x64, accumulators in
//    VGPRs or, as inline asm, in AGPRs) and time themselves in shader-clock
//    cycles and in the 100 MHz real-time counter; meanwhile waves 4-7 idle
//    (busy = 0), run independent v_fma_f32 streams long enough to outlast
//    them (busy = 1), issue the same MFMA stream (busy = 2), or stream
//    conflict-free 128-bit LDS reads (busy = 3: 1 KB per instruction, eight
//    in flight per wave), or run independent v_exp_f32 (busy = 4) or
//    v_dot2_f32_bf16 (busy = 5) streams, the attention softmax's
//    transcendental and row-sum instructions.  Each wave
//    records its hardware id, so the host can check that waves w and w + 4
//    share a SIMD.
//  * mxp_promote_launch: the fp8 GEMM's block promotion.  Every wave keeps
//    8 fp32 accumulators of 32x32 and per iteration, for each, builds a
//    fresh partial from two 32x32x64 fp8 MFMAs (one 128-deep scale block)
//    and promotes it, acc += s * partial (16 v_fma per lane); the partials
//    rotate through NP registers sets, and the promotion of fragment f runs
//    after the MFMAs of fragment f + LAG, in the compiler's order or in an
//    enforced one.  Variants: no promotion (the MFMAs accumulate straight
//    into the accumulators), alone or beside the same FMAs on registers no
//    MFMA writes.  One workgroup per CU of 4 waves (one per
//    SIMD) or 8 (two per SIMD); shader-clock cycles per wave.
//  * mxp_wg_read_launch: nwg workgroups of 256 threads; workgroup w reads n16
//    16-byte elements starting at element w * stride16 (eight loads in
//    flight per thread) and writes one XOR per thread, so the time of a
//    launch against an empty one gives the read bandwidth of that many
//    workgroups.
//  * mxp_stream_launch: the same reads with a chosen number in flight, as
//    loads into registers (DEPTH per thread, consumed as a batch) or as
//    direct global -> LDS loads (global_load_lds_dwordx4, the kernels' tile
//    copies: 1 KB per wave instruction, DEPTH of them in flight per wave
//    through a ring of DEPTH KB), so the time of a launch gives a
//    workgroup's read rate against the bytes it keeps in flight.
#include <type_traits>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "mx_common.h"

namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kOverlapLds = 150 * 1024;
constexpr int kOverlapThreads = 256;

// The mix beside MFMA m of an iteration (32 independent registers e / u).
template <int OP>
__device__ __forceinline__ void mix(float* e, unsigned* u, int m) {
  if constexpr (OP == 9) {  // the v_exp_f32 mix with an s_nop 1 after each MFMA
    asm volatile("s_nop 1");
#pragma unroll
    for (int j = 0; j < 4; ++j) e[4 * m + j] = __builtin_amdgcn_exp2f(e[4 * m + j]);
  } else if constexpr (OP == 7) {
    asm volatile("s_nop 0");
  } else if constexpr (OP == 8) {
    asm volatile("s_nop 1");
  } else {
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3f803f80u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * m + j;
      if constexpr (OP == 1) e[i] = __builtin_amdgcn_exp2f(e[i]);
      if constexpr (OP == 2)  // the previous pack's bits feed the next (one instruction, loop-carried)
        u[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{e[i], __builtin_bit_cast(float, u[i])}, bf16x2));
      if constexpr (OP == 3) e[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u[i]), ones, e[i], false);
      if constexpr (OP == 4) e[i] = e[i] + e[i ^ 2];
      if constexpr (OP == 5) e[i] = e[i] * e[i ^ 2];
      if constexpr (OP == 6) e[i] = __builtin_fmaf(e[i], 0.999f, e[i ^ 2]);
    }
  }
}

template <int OP, bool MF>
__global__ __launch_bounds__(kOverlapThreads, 1) void overlap_kernel(float* out, long long* cycles, int iters) {
  extern __shared__ char lds[];
  lds[threadIdx.x] = 0;
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{} + 1e-3f * i;
  const u32x4 a = u32x4{threadIdx.x, 7u, 9u, 11u}, b = u32x4{3u, threadIdx.x, 5u, 13u};
  float e[32];
  unsigned u[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    e[i] = 1e-6f * (threadIdx.x + i);
    u[i] = threadIdx.x * 7u + i;
  }
  // OP 10: each MFMA's B operand is a 128-bit LDS read (1 KB per wave,
  // lane i reading bytes 16 i .. 16 i + 15: conflict-free) issued one
  // iteration ahead, as the kernels read their fragments; without MFMAs the
  // reads are consumed by one v_xor each.  Each wave reads its own 32 KB.
  u32x4 v[8];
  const u32x4* lb = reinterpret_cast<const u32x4*>(lds) + (threadIdx.x >> 6) * 2048;
  if constexpr (OP == 10) {
    u32x4* lw = reinterpret_cast<u32x4*>(lds) + (threadIdx.x >> 6) * 2048;
    for (int i = threadIdx.x & 63; i < 2048; i += 64) lw[i] = u32x4{0x3f803f80u ^ (unsigned)i, 0x3e003e00u, 0x3f003f00u, (unsigned)i};
#pragma unroll
    for (int m = 0; m < 8; ++m) v[m] = lb[m * 64 + (threadIdx.x & 63)];
  }
  const long long t0 = __builtin_readcyclecounter();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if constexpr (OP == 10) {
        if constexpr (MF)
          acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                           __builtin_bit_cast(bf16x8, v[m]), acc[m], 0, 0, 0);
        else
          u[m] ^= v[m][0];
        v[m] = lb[(((it + 1) * 8 + m) & 31) * 64 + (threadIdx.x & 63)];
      } else {
        if constexpr (MF)
          acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                           acc[m], 0, 0, 0);
        mix<OP>(e, u, m);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const long long t1 = __builtin_readcyclecounter();
  if constexpr (OP == 10) {
#pragma unroll
    for (int m = 0; m < 8; ++m) u[m] ^= v[m][1];
  }
  float r = 0.f;
#pragma unroll
  for (int m = 0; m < 8; ++m) r += acc[m][threadIdx.x & 15];
#pragma unroll
  for (int i = 0; i < 32; ++i) r += e[i] + (float)u[i];
  out[blockIdx.x * kOverlapThreads + threadIdx.x] = r + lds[(threadIdx.x * 7) & 255];
  if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
}

// HIP errors come back as -(1000 + hipError_t); mxp_error_string names them.
int hip_status(hipError_t e) { return e == hipSuccess ? 0 : -(1000 + (int)e); }

template <int OP, bool MF>
int launch_overlap(int nwg, int iters, float* out, long long* cycles, hipStream_t s) {
  constexpr auto k = overlap_kernel<OP, MF>;
  if (const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kOverlapLds);
      e != hipSuccess)
    return hip_status(e);
  hipLaunchKernelGGL(k, dim3(nwg), dim3(kOverlapThreads), kOverlapLds, s, out, cycles, iters);
  return hip_status(hipGetLastError());
}

template <int OP>
int launch_op(int with_mfma, int nwg, int iters, float* out, long long* cycles, hipStream_t s) {
  return with_mfma ? launch_overlap<OP, true>(nwg, iters, out, cycles, s)
                   : launch_overlap<OP, false>(nwg, iters, out, cycles, s);
}

constexpr int kRateWaves = 8;

// 8 accumulators per wave; MFMA j of an iteration takes A fragment j % 4 and
// B fragment (j / 2) % 4, so consecutive MFMAs differ in an operand.
// SHAPE 0: 32x32x16 bf16 (VGPR accumulators), 1: 16x16x32 bf16, 2: 32x32x16
// bf16 with AGPR accumulators, 3: 32x32x64 fp8 e4m3, 4: 16x16x128 fp8 e4m3
// (the fp8 ones in the scaled form with unit scales, as the kernels issue
// them; a 32-byte operand is two of the 16-byte fragments); with AGPR
// accumulators (inline asm): 5: 16x16x32 bf16, 6: 32x32x64 fp8, 7:
// 16x16x128 fp8.
template <int SHAPE>
__global__ __launch_bounds__(64 * kRateWaves, 1) void mfma_rate_kernel(const u32x4* __restrict__ ops, float* out,
                                                                      int iters) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = ops[t * 8 + j];
    b[j] = ops[t * 8 + 4 + j];
  }
  float r = 0.f;
  if constexpr (SHAPE == 2) {
    // inline asm keeps the accumulators in AGPRs; 21 wait states before they
    // are read back (the compiler does not guard asm MFMAs)
    f32x16 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a[j & 3]), "v"(b[(j >> 1) & 3]));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(acc[j]));
#pragma unroll
    for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 15];
  } else if constexpr (SHAPE == 5) {
    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a[j & 3]), "v"(b[(j >> 1) & 3]));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("s_nop 7\n\ts_nop 3" : "+a"(acc[j]));
#pragma unroll
    for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 3];
  } else if constexpr (SHAPE == 6 || SHAPE == 7) {
    typedef int i32x8 __attribute__((ext_vector_type(8)));
    i32x8 a8[4], b8[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 a0 = a[j], a1 = a[(j + 1) & 3], b0 = b[j], b1 = b[(j + 1) & 3];
      a8[j] = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
      b8[j] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    }
    if constexpr (SHAPE == 6) {
      f32x16 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          asm("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a8[j & 3]), "v"(b8[(j >> 1) & 3]));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(acc[j]));
#pragma unroll
      for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 15];
    } else {
      f32x4 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = f32x4{};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          asm("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a8[j & 3]), "v"(b8[(j >> 1) & 3]));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) asm volatile("s_nop 7\n\ts_nop 3" : "+a"(acc[j]));
#pragma unroll
      for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 3];
    }
  } else if constexpr (SHAPE == 3 || SHAPE == 4) {
    typedef int i32x8 __attribute__((ext_vector_type(8)));
    i32x8 a8[4], b8[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 a0 = a[j], a1 = a[(j + 1) & 3], b0 = b[j], b1 = b[(j + 1) & 3];
      a8[j] = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
      b8[j] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    }
    if constexpr (SHAPE == 3) {
      f32x16 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8[j & 3], b8[(j >> 1) & 3], acc[j], 0, 0, 0, 127,
                                                                   0, 127);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 15];
    } else {
      f32x4 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = f32x4{};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8[j & 3], b8[(j >> 1) & 3], acc[j], 0, 0, 0, 127,
                                                                    0, 127);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 3];
    }
  } else if constexpr (SHAPE == 0) {
    f32x16 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[j & 3]),
                                                         __builtin_bit_cast(bf16x8, b[(j >> 1) & 3]), acc[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 15];
  } else {
    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[j & 3]),
                                                         __builtin_bit_cast(bf16x8, b[(j >> 1) & 3]), acc[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 3];
  }
  out[t] = r;
}

__global__ __launch_bounds__(256) void wg_read_kernel(const uint4* __restrict__ src, long long stride16, long long n16,
                                                     unsigned* out) {
  const uint4* p = src + blockIdx.x * stride16;
  unsigned acc = 0;
  for (long long i = threadIdx.x; i < n16; i += 256 * 8) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const long long k = i + (long long)j * 256;
      v[j] = k < n16 ? p[k] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

// FORM 0: bf16 32x32x16, VGPR accumulators; 1: the same in AGPRs (asm);
// 2: fp8 e4m3 32x32x64, VGPR accumulators (the scaled form with unit
// scales, as the kernels issue it); 3: fp8 32x32x64 in AGPRs (asm); 4: bf16
// 16x16x32, VGPR accumulators (the bf16 GEMMs' shape).
// cycles[8 b + w], rtime[8 b + w] (waves 4-7 only with busy > 0) and
// hwid[8 b + w] per wave w of workgroup b.
template <int FORM, int BUSY>
__global__ __launch_bounds__(512, 1) void contend_kernel(const u32x4* __restrict__ ops, float* out, long long* cycles,
                                                        long long* rtime, unsigned* hwid, int iters,
                                                        int valu_iters) {
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if ((threadIdx.x & 63) == 0) hwid[blockIdx.x * 8 + wave] = __builtin_amdgcn_s_getreg((31 << 11) | 4);
  float r = 0.f;
  if (wave < 4 || BUSY == 2) {
    u32x4 a[2], b[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      a[j] = ops[t * 4 + j];
      b[j] = ops[t * 4 + 2 + j];
    }
    const i32x8 a8 = __builtin_bit_cast(i32x8, (u32x4[2]){a[0], a[1]});
    const i32x8 b8 = __builtin_bit_cast(i32x8, (u32x4[2]){b[0], b[1]});
    using Acc = std::conditional_t<FORM == 4, f32x4_t, f32x16>;
    Acc acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = Acc{};
    const long long r0 = __builtin_amdgcn_s_memrealtime();
    const long long t0 = __builtin_readcyclecounter();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (FORM == 4)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[j & 1]),
                                                           __builtin_bit_cast(bf16x8, b[(j >> 1) & 1]), acc[j], 0, 0, 0);
        else if constexpr (FORM == 0)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[j & 1]),
                                                           __builtin_bit_cast(bf16x8, b[(j >> 1) & 1]), acc[j], 0, 0, 0);
        else if constexpr (FORM == 1)
          asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a[j & 1]), "v"(b[(j >> 1) & 1]));
        else if constexpr (FORM == 2)
          acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[j], 0, 0, 0, 127, 0, 127);
        else
          asm("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+a"(acc[j]) : "v"(a8), "v"(b8));
      }
    }
    const long long t1 = __builtin_readcyclecounter();
    const long long r1 = __builtin_amdgcn_s_memrealtime();
    if constexpr (FORM == 1 || FORM == 3) {
#pragma unroll
      for (int j = 0; j < 8; ++j) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(acc[j]));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & (FORM == 4 ? 3 : 15)];
    if ((threadIdx.x & 63) == 0) {
      cycles[blockIdx.x * 8 + wave] = t1 - t0;
      rtime[blockIdx.x * 8 + wave] = r1 - r0;
    }
  } else if constexpr (BUSY == 3) {
    // waves 4-7 read their own 16 KB of LDS: lane i reads bytes 16 i ..
    // 16 i + 15 of a 1 KB block (16 distinct 16-byte slots per 16-lane
    // group: no bank conflicts), eight blocks per iteration
    __shared__ u32x4 lbuf[4 * 1024];
    u32x4* mine = lbuf + (wave - 4) * 1024;
    const int lane = threadIdx.x & 63;
    for (int i = lane; i < 1024; i += 64) mine[i] = u32x4{(unsigned)i, (unsigned)t, 1u, 2u};
    u32x4 x = u32x4{0u, 0u, 0u, 0u};
    const long long r0 = __builtin_amdgcn_s_memrealtime();
    const long long t0 = __builtin_readcyclecounter();
    for (int it = 0; it < valu_iters; ++it) {
      asm volatile("" ::: "memory");  // every iteration reads LDS again
      u32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = mine[((it * 8 + j) & 15) * 64 + lane];
#pragma unroll
      for (int j = 0; j < 8; ++j) x ^= v[j];
    }
    const long long t1 = __builtin_readcyclecounter();
    const long long r1 = __builtin_amdgcn_s_memrealtime();
    r += (float)(x[0] ^ x[1] ^ x[2] ^ x[3]);
    if (lane == 0) {
      cycles[blockIdx.x * 8 + wave] = t1 - t0;
      rtime[blockIdx.x * 8 + wave] = r1 - r0;
    }
  } else if constexpr (BUSY == 1 || BUSY == 4 || BUSY == 5) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    float e[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) e[i] = 1e-6f * (threadIdx.x + i);
    const bf2 p2{(__bf16)1e-6f, (__bf16)2e-6f}, ones{(__bf16)1.0f, (__bf16)1.0f};
    const long long r0 = __builtin_amdgcn_s_memrealtime();
    const long long t0 = __builtin_readcyclecounter();
    for (int it = 0; it < valu_iters; ++it) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        if constexpr (BUSY == 1)
          e[i] = __builtin_fmaf(e[i], 0.999f, e[i ^ 2]);
        else if constexpr (BUSY == 4)
          e[i] = __builtin_amdgcn_exp2f(-e[i]);  // stays in (0, 1]
        else
          e[i] = __builtin_amdgcn_fdot2_f32_bf16(p2, ones, e[i], false);
      }
    }
    const long long t1 = __builtin_readcyclecounter();
    const long long r1 = __builtin_amdgcn_s_memrealtime();
#pragma unroll
    for (int i = 0; i < 32; ++i) r += e[i];
    if ((threadIdx.x & 63) == 0) {
      cycles[blockIdx.x * 8 + wave] = t1 - t0;
      rtime[blockIdx.x * 8 + wave] = r1 - r0;
    }
  }
  out[t] = r;
}

template <int FORM>
int launch_contend(int busy, int nwg, int iters, int valu_iters, const u32x4* ops, float* out, long long* cycles,
                   long long* rtime, unsigned* hwid, hipStream_t s) {
  if (busy == 0)
    hipLaunchKernelGGL((contend_kernel<FORM, 0>), dim3(nwg), dim3(512), 0, s, ops, out, cycles, rtime, hwid, iters,
                       valu_iters);
  else if (busy == 1)
    hipLaunchKernelGGL((contend_kernel<FORM, 1>), dim3(nwg), dim3(512), 0, s, ops, out, cycles, rtime, hwid, iters,
                       valu_iters);
  else if (busy == 2)
    hipLaunchKernelGGL((contend_kernel<FORM, 2>), dim3(nwg), dim3(512), 0, s, ops, out, cycles, rtime, hwid, iters,
                       valu_iters);
  else if (busy == 3)
    hipLaunchKernelGGL((contend_kernel<FORM, 3>), dim3(nwg), dim3(512), 0, s, ops, out, cycles, rtime, hwid, iters,
                       valu_iters);
  else if (busy == 4)
    hipLaunchKernelGGL((contend_kernel<FORM, 4>), dim3(nwg), dim3(512), 0, s, ops, out, cycles, rtime, hwid, iters,
                       valu_iters);
  else
    hipLaunchKernelGGL((contend_kernel<FORM, 5>), dim3(nwg), dim3(512), 0, s, ops, out, cycles, rtime, hwid, iters,
                       valu_iters);
  return hip_status(hipGetLastError());
}

// MODE 0: no promotion; 1: acc += s * partial, the partial of fragment f
// promoted after the MFMAs of fragment f + LAG (NP = LAG + 1 partial sets,
// rounded up to a divisor of 8), in the compiler's order; 3: the same with
// that order enforced (scheduling groups: the fragment's two MFMAs, then the
// 16 FMAs); 2: mode 0's MFMAs plus the same FMAs on registers no MFMA
// writes.  cycles[b * NW + w].
template <int MODE, int LAG, int NW>
__global__ __launch_bounds__(64 * NW, 2) void promote_kernel(const u32x4* __restrict__ ops, float* out,
                                                            long long* cycles, int iters) {
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  constexpr int NP = LAG + 1 <= 2 ? 2 : (LAG + 1 <= 4 ? 4 : 8);
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 q[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) q[j] = ops[t * 4 + j];
  i32x8 a8 = __builtin_bit_cast(i32x8, (u32x4[2]){q[0], q[1]});
  const i32x8 b8 = __builtin_bit_cast(i32x8, (u32x4[2]){q[2], q[3]});
  const float sc = 1.0f + 1e-3f * (float)(threadIdx.x & 7);
  f32x16 acc[8], part[NP];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
#pragma unroll
  for (int j = 0; j < NP; ++j) part[j] = f32x16{} + 1e-3f * j;
  auto promote = [&](int f) {
    const f32x16& p = part[f % NP];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[f][e] = __builtin_fmaf(sc, p[e], acc[f][e]);
  };
  const long long t0 = __builtin_readcyclecounter();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      // an empty statement that the compiler must assume rewrote the operand,
      // so no fragment's fresh partial is hoisted out of the loop or shared
      asm volatile("" : "+v"(a8));
      if constexpr (MODE == 0 || MODE == 2) {
        acc[f] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[f], 0, 0, 0, 127, 0, 127);
        acc[f] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b8, a8, acc[f], 0, 0, 0, 127, 0, 127);
        if constexpr (MODE == 2) {
          const f32x16& r = part[f % NP];
#pragma unroll
          for (int e = 0; e < 16; ++e) part[(f + 1) % NP][e] = __builtin_fmaf(sc, r[e], part[(f + 1) % NP][e]);
        }
      } else {
        f32x16 p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, f32x16{}, 0, 0, 0, 127, 0, 127);
        p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b8, a8, p, 0, 0, 0, 127, 0, 127);
        part[f % NP] = p;
        if (f >= LAG) promote(f - LAG);
        if constexpr (MODE == 3) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          if (f >= LAG) __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
        }
      }
    }
    if constexpr (MODE == 1 || MODE == 3) {
#pragma unroll
      for (int f = 8 - LAG; f < 8; ++f) promote(f);
    }
  }
  const long long t1 = __builtin_readcyclecounter();
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) r += acc[j][threadIdx.x & 15];
#pragma unroll
  for (int j = 0; j < NP; ++j) r += part[j][threadIdx.x & 15];
  out[t] = r;
  if ((threadIdx.x & 63) == 0) cycles[blockIdx.x * NW + wave] = t1 - t0;
}

template <int MODE, int LAG, int NW>
int launch_promote(int nwg, int iters, const u32x4* ops, float* out, long long* cycles, hipStream_t s) {
  hipLaunchKernelGGL((promote_kernel<MODE, LAG, NW>), dim3(nwg), dim3(64 * NW), 0, s, ops, out, cycles, iters);
  return hip_status(hipGetLastError());
}

template <int MODE, int NW>
int launch_promote_lag(int lag, int nwg, int iters, const u32x4* ops, float* out, long long* cycles, hipStream_t s) {
  switch (lag) {
    case 1: return launch_promote<MODE, 1, NW>(nwg, iters, ops, out, cycles, s);
    case 2: return launch_promote<MODE, 2, NW>(nwg, iters, ops, out, cycles, s);
    default: return launch_promote<MODE, 3, NW>(nwg, iters, ops, out, cycles, s);
  }
}

template <int DEPTH>
__global__ __launch_bounds__(256) void stream_reg_kernel(const uint4* __restrict__ src, long long stride16,
                                                        long long n16, unsigned* out) {
  const uint4* p = src + blockIdx.x * stride16;
  unsigned acc = 0;
  for (long long i = threadIdx.x; i < n16; i += 256 * DEPTH) {
    uint4 v[DEPTH];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) {
      const long long k = i + (long long)j * 256;
      v[j] = k < n16 ? p[k] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

// Wave w copies the 1 KB chunks w, w + 4, ... of its workgroup's n16
// elements (n16 % 64 == 0) into ring slot c % DEPTH of its own DEPTH KB,
// where c counts its chunks; before reusing a slot it waits until at most
// DEPTH - 1 of its loads are outstanding, i.e. the slot's previous load has
// landed.
template <int DEPTH>
__global__ __launch_bounds__(256) void stream_lds_kernel(const uint4* __restrict__ src, long long stride16,
                                                        long long n16, unsigned* out) {
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint4* p = src + blockIdx.x * stride16;
  const uint32_t ring = mx::lds_addr(smem) + wave * DEPTH * 1024;
  const long long chunks = n16 / 64;
  int c = 0;
  for (long long k = wave; k < chunks; k += 4, ++c) {
    if (c >= DEPTH) mx::wait_vmcnt<DEPTH - 1>();
    mx::dma16(p + k * 64, 16u * lane, ring + (c % DEPTH) * 1024);
  }
  mx::wait_vmcnt<0>();
  __syncthreads();
  out[blockIdx.x * 256 + threadIdx.x] = reinterpret_cast<const unsigned*>(smem)[threadIdx.x];
}

template <int MODE, int DEPTH>
int launch_stream(const uint4* src, long long stride16, long long n16, int nwg, unsigned* out, hipStream_t s) {
  if constexpr (MODE == 0) {
    hipLaunchKernelGGL(stream_reg_kernel<DEPTH>, dim3(nwg), dim3(256), 0, s, src, stride16, n16, out);
  } else {
    constexpr int lds = 4 * DEPTH * 1024;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(stream_lds_kernel<DEPTH>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return hip_status(e);
    hipLaunchKernelGGL(stream_lds_kernel<DEPTH>, dim3(nwg), dim3(256), lds, s, src, stride16, n16, out);
  }
  return hip_status(hipGetLastError());
}

}  // namespace

// probe: 0 MFMAs only, 1 v_exp_f32, 2 v_cvt_pk_bf16_f32, 3 v_dot2_f32_bf16,
// 4 v_add_f32, 5 v_mul_f32, 6 v_fma_f32 (32 per iteration), 7 s_nop 0,
// 8 s_nop 1 (one per MFMA), 9 the v_exp_f32 mix with an s_nop 1 per MFMA,
// 10 eight 128-bit LDS reads, each the B operand of the next iteration's
// MFMA (without MFMAs: consumed by one v_xor each).  out: nwg * 256 floats; cycles: nwg entries.
// Returns 0, -1 for invalid arguments or an unknown probe, or -(1000 + e)
// for HIP error e.
extern "C" int mxp_overlap_launch(int probe, int with_mfma, int nwg, int iters, float* out, long long* cycles,
                                  void* stream) {
  if (nwg <= 0 || iters <= 0 || !out || !cycles) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (probe) {
    case 0: return launch_op<0>(1, nwg, iters, out, cycles, s);
    case 1: return launch_op<1>(with_mfma, nwg, iters, out, cycles, s);
    case 2: return launch_op<2>(with_mfma, nwg, iters, out, cycles, s);
    case 3: return launch_op<3>(with_mfma, nwg, iters, out, cycles, s);
    case 4: return launch_op<4>(with_mfma, nwg, iters, out, cycles, s);
    case 5: return launch_op<5>(with_mfma, nwg, iters, out, cycles, s);
    case 6: return launch_op<6>(with_mfma, nwg, iters, out, cycles, s);
    case 7: return launch_op<7>(with_mfma, nwg, iters, out, cycles, s);
    case 8: return launch_op<8>(with_mfma, nwg, iters, out, cycles, s);
    case 9: return launch_op<9>(with_mfma, nwg, iters, out, cycles, s);
    case 10: return launch_op<10>(with_mfma, nwg, iters, out, cycles, s);
    default: return -1;
  }
}

// shape 0: 32x32x16, 1: 16x16x32, 2: 32x32x16 with AGPR accumulators (bf16);
// 3: 32x32x64, 4: 16x16x128 (fp8 e4m3); AGPR accumulators: 5: 16x16x32
// bf16, 6: 32x32x64 fp8, 7: 16x16x128 fp8.  ops: nwg * 512 * 8 16-byte
// fragments (lane t of the grid reads its 8 at 8 t); out: nwg * 512 floats.
// FLOPs of a launch: nwg * 8 waves * iters * 8 MFMAs * 32768 (shapes 0, 2),
// 16384 (1, 5), 131072 (3, 6) or 65536 (4, 7).  The builtins (shapes 0, 1,
// 3, 4) get VGPR accumulators from this compiler at two waves per SIMD.
extern "C" int mxp_mfma_rate_launch(int shape, int nwg, int iters, const void* ops, float* out, void* stream) {
  if (nwg <= 0 || iters <= 0 || !ops || !out || shape < 0 || shape > 7) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* o = static_cast<const u32x4*>(ops);
  const dim3 grid(nwg), block(64 * kRateWaves);
  switch (shape) {
    case 0: hipLaunchKernelGGL(mfma_rate_kernel<0>, grid, block, 0, s, o, out, iters); break;
    case 1: hipLaunchKernelGGL(mfma_rate_kernel<1>, grid, block, 0, s, o, out, iters); break;
    case 2: hipLaunchKernelGGL(mfma_rate_kernel<2>, grid, block, 0, s, o, out, iters); break;
    case 3: hipLaunchKernelGGL(mfma_rate_kernel<3>, grid, block, 0, s, o, out, iters); break;
    case 4: hipLaunchKernelGGL(mfma_rate_kernel<4>, grid, block, 0, s, o, out, iters); break;
    case 5: hipLaunchKernelGGL(mfma_rate_kernel<5>, grid, block, 0, s, o, out, iters); break;
    case 6: hipLaunchKernelGGL(mfma_rate_kernel<6>, grid, block, 0, s, o, out, iters); break;
    default: hipLaunchKernelGGL(mfma_rate_kernel<7>, grid, block, 0, s, o, out, iters); break;
  }
  return hip_status(hipGetLastError());
}

// src must hold (nwg - 1) * stride16 + n16 16-byte elements; out nwg * 256.
extern "C" int mxp_wg_read_launch(const void* src, long long stride16, long long n16, int nwg, unsigned* out,
                                  void* stream) {
  if (nwg <= 0 || n16 < 0 || stride16 < 0 || !src || !out) return -1;
  hipLaunchKernelGGL(wg_read_kernel, dim3(nwg), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), stride16, n16, out);
  return hip_status(hipGetLastError());
}

// mode 0: loads into registers, depth 4, 8, 16 or 32 per thread; mode 1:
// direct LDS loads, depth 4, 8, 16 or 32 KB in flight per wave (n16 a
// multiple of 64).  src must hold (nwg - 1) * stride16 + n16 16-byte
// elements; out nwg * 256.
extern "C" int mxp_stream_launch(int mode, int depth, const void* src, long long stride16, long long n16, int nwg,
                                 unsigned* out, void* stream) {
  if (nwg <= 0 || n16 < 0 || stride16 < 0 || !src || !out || mode < 0 || mode > 1) return -1;
  if (mode == 1 && n16 % 64 != 0) return -1;
  const uint4* p = static_cast<const uint4*>(src);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (mode * 100 + depth) {
    case 4: return launch_stream<0, 4>(p, stride16, n16, nwg, out, s);
    case 8: return launch_stream<0, 8>(p, stride16, n16, nwg, out, s);
    case 16: return launch_stream<0, 16>(p, stride16, n16, nwg, out, s);
    case 32: return launch_stream<0, 32>(p, stride16, n16, nwg, out, s);
    case 104: return launch_stream<1, 4>(p, stride16, n16, nwg, out, s);
    case 108: return launch_stream<1, 8>(p, stride16, n16, nwg, out, s);
    case 116: return launch_stream<1, 16>(p, stride16, n16, nwg, out, s);
    case 132: return launch_stream<1, 32>(p, stride16, n16, nwg, out, s);
    default: return -1;
  }
}

// form 0..4 as contend_kernel; busy 0 (waves 4-7 idle), 1 (VALU), 2 (the
// same MFMAs), 3 (LDS reads; valu_iters iterations of eight 1 KB reads), 4
// (v_exp_f32) or 5 (v_dot2_f32_bf16; 4 and 5 as 1: 32 chains per lane).  ops: nwg * 512 * 4 16-byte fragments (lane t reads its
// 4 at 4 t); out: nwg * 512 floats; cycles, rtime and hwid: nwg * 8 each.
extern "C" int mxp_contend_launch(int form, int busy, int nwg, int iters, int valu_iters, const void* ops, float* out,
                                  long long* cycles, long long* rtime, unsigned* hwid, void* stream) {
  if (nwg <= 0 || iters <= 0 || valu_iters < 0 || !ops || !out || !cycles || !rtime || !hwid || form < 0 ||
      form > 4 || busy < 0 || busy > 5)
    return -1;
  const u32x4* o = static_cast<const u32x4*>(ops);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (form) {
    case 0: return launch_contend<0>(busy, nwg, iters, valu_iters, o, out, cycles, rtime, hwid, s);
    case 1: return launch_contend<1>(busy, nwg, iters, valu_iters, o, out, cycles, rtime, hwid, s);
    case 2: return launch_contend<2>(busy, nwg, iters, valu_iters, o, out, cycles, rtime, hwid, s);
    case 3: return launch_contend<3>(busy, nwg, iters, valu_iters, o, out, cycles, rtime, hwid, s);
    default: return launch_contend<4>(busy, nwg, iters, valu_iters, o, out, cycles, rtime, hwid, s);
  }
}

// mode 0..3 as promote_kernel; lag 1..3 (modes 1 and 3); waves 4 or 8 per
// workgroup.  ops: nwg * 64 * waves * 4 16-byte fragments (lane t reads its 4
// at 4 t); out: nwg * 64 * waves floats; cycles: nwg * waves.
extern "C" int mxp_promote_launch(int mode, int lag, int waves, int nwg, int iters, const void* ops, float* out,
                                  long long* cycles, void* stream) {
  if (nwg <= 0 || iters <= 0 || !ops || !out || !cycles || mode < 0 || mode > 3 || (waves != 4 && waves != 8) ||
      ((mode == 1 || mode == 3) && (lag < 1 || lag > 3)))
    return -1;
  const u32x4* o = static_cast<const u32x4*>(ops);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool two = waves == 8;
  switch (mode) {
    case 0: return two ? launch_promote<0, 1, 8>(nwg, iters, o, out, cycles, s)
                       : launch_promote<0, 1, 4>(nwg, iters, o, out, cycles, s);
    case 2: return two ? launch_promote<2, 1, 8>(nwg, iters, o, out, cycles, s)
                       : launch_promote<2, 1, 4>(nwg, iters, o, out, cycles, s);
    case 1: return two ? launch_promote_lag<1, 8>(lag, nwg, iters, o, out, cycles, s)
                       : launch_promote_lag<1, 4>(lag, nwg, iters, o, out, cycles, s);
    default: return two ? launch_promote_lag<3, 8>(lag, nwg, iters, o, out, cycles, s)
                        : launch_promote_lag<3, 4>(lag, nwg, iters, o, out, cycles, s);
  }
}

// The HIP error behind a status below -1000.
extern "C" const char* mxp_error_string(int status) {
  return status <= -1000 ? hipGetErrorString(static_cast<hipError_t>(-status - 1000)) : "invalid argument";
}
