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
//  * mxp_wg_read_launch: nwg workgroups of 256 threads; workgroup w reads n16
//    16-byte elements starting at element w * stride16 (eight loads in
//    flight per thread) and writes one XOR per thread, so the time of a
//    launch against an empty one gives the read bandwidth of that many
//    workgroups.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

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
  const long long t0 = __builtin_readcyclecounter();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if constexpr (MF)
        acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                         acc[m], 0, 0, 0);
      mix<OP>(e, u, m);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const long long t1 = __builtin_readcyclecounter();
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

}  // namespace

// probe: 0 MFMAs only, 1 v_exp_f32, 2 v_cvt_pk_bf16_f32, 3 v_dot2_f32_bf16,
// 4 v_add_f32, 5 v_mul_f32, 6 v_fma_f32 (32 per iteration), 7 s_nop 0,
// 8 s_nop 1 (one per MFMA), 9 the v_exp_f32 mix with an s_nop 1 per MFMA.  out: nwg * 256 floats; cycles: nwg entries.
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
    default: return -1;
  }
}

// src must hold (nwg - 1) * stride16 + n16 16-byte elements; out nwg * 256.
extern "C" int mxp_wg_read_launch(const void* src, long long stride16, long long n16, int nwg, unsigned* out,
                                  void* stream) {
  if (nwg <= 0 || n16 < 0 || stride16 < 0 || !src || !out) return -1;
  hipLaunchKernelGGL(wg_read_kernel, dim3(nwg), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), stride16, n16, out);
  return hip_status(hipGetLastError());
}

// The HIP error behind a status below -1000.
extern "C" const char* mxp_error_string(int status) {
  return status <= -1000 ? hipGetErrorString(static_cast<hipError_t>(-status - 1000)) : "invalid argument";
}
