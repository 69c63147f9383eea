// Shared device helpers for the gfx950 (CDNA4) kernels of this library.
//
// Everything here is written for one target: gfx950, wave64, MFMA matrix
// cores, 160 KB LDS per CU.  There is no other code path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "mx_kernels.h"

namespace mx {

// ---------------------------------------------------------------------------
// Vector types used as MFMA operands / accumulators and for 128-bit traffic.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Conversions.  Narrowing to bf16 / f16 uses gfx950's packed converts
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: two fp32 -> two 16-bit values in
// one instruction, round-to-nearest-even), the same rounding torch's CPU
// cast applies, so device outputs are comparable bit-for-bit with a host
// cast of the same fp32 value.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Pack two fp32 into one dword of two bf16 (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)x;
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

// Element-type tags for the 16-bit I/O formats the kernels accept.
struct BF16 {
  static __device__ __forceinline__ float to_f32(uint32_t h) { return bf16_bits_to_f32(h); }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) { return pack_bf16x2(a, b); }
};
struct F16 {
  static __device__ __forceinline__ float to_f32(uint32_t h) { return f16_bits_to_f32(h); }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) { return pack_f16x2(a, b); }
};

// ---------------------------------------------------------------------------
// MFMA wrappers.  Operand register images are passed as raw dwords so the
// same staging code serves bf16 and f16.
//
// Lane layouts assumed (CDNA3/CDNA4 MFMA, wave64):
//   16x16x32 (bf16/f16): A: lane l holds row l%16, k = 8*(l/16) .. +7
//                        B: lane l holds col l%16, k = 8*(l/16) .. +7
//                        D: lane l holds col l%16, rows 4*(l/16) .. +3
//   32x32x16 (bf16/f16): A: lane l holds row l%32, k = 8*(l/32) .. +7
//                        B: lane l holds col l%32, k = 8*(l/32) .. +7
//                        D: lane l holds col l%32,
//                           rows 8*i + 4*(l/32) + j  for acc[4*i + j]
// A contraction only needs A and B to agree on which k each register
// position carries, so kernels are free to permute k consistently.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c);
template <>
__device__ __forceinline__ f32x4 mfma16<BF16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<F16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c);
template <>
__device__ __forceinline__ f32x16 mfma32<BF16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<F16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// fp8 e4m3 (OCP "fn" encoding on gfx950) x e4m3 -> fp32, 16x16x128.
// Issued through the block-scaled form with both E8M0 scales = 127 (2^0),
// i.e. an unscaled product.  A: lane l holds row l%16 and 32 k-bytes,
// B: lane l holds col l%16 and the same 32 k positions.
__device__ __forceinline__ f32x4 mfma16_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// acc += a·b on a 32x32x16 MFMA whose accumulator stays in AGPRs.  The
// builtin MFMAs of a kernel all take one register class, chosen by the
// compiler; issuing this one as inline asm keeps its accumulator in AGPRs
// while the kernel's other MFMAs write VGPRs.  The compiler does not know
// the asm is an MFMA and inserts none of the wait states around it: any
// other reader or writer of the accumulator calls agpr_settle() first, and
// a VALU-written A or B operand goes through operand_settle() (two wait
// states) before the MFMA reads it; the build check of the assembly asserts
// both (an `s_nop` in front of every MFMA would cost ~7 cycles each in a
// stream of MFMAs).  Back-to-back accumulation into the same registers needs no
// wait states.
template <typename T>
__device__ __forceinline__ void mfma32_agpr(f32x16& acc, const u32x4& a, const u32x4& b);
template <>
__device__ __forceinline__ void mfma32_agpr<BF16>(f32x16& acc, const u32x4& a, const u32x4& b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
template <>
__device__ __forceinline__ void mfma32_agpr<F16>(f32x16& acc, const u32x4& a, const u32x4& b) {
  asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Two wait states after the VALU writes that produced x, before an
// mfma32_agpr reads it as an operand.  x is an operand of the wait, so the
// MFMAs that read it cannot be scheduled above it, and no VALU write to it
// can follow it.
__device__ __forceinline__ void operand_settle(u32x4& x) { asm volatile("s_nop 1" : "+v"(x)); }

// 21 wait states after the last mfma32_agpr into acc, before any other
// instruction reads or writes those AGPRs (a 32x32 MFMA's result needs up
// to 19 before a VALU or v_accvgpr_* access).  acc is an operand, so the
// accesses that follow cannot be scheduled above it.
__device__ __forceinline__ void agpr_settle(f32x16& acc) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(acc));
}

// acc *= c for an accumulator held in AGPRs: read, multiply, write back one
// register at a time (VALU cannot read AGPRs), without ever materialising
// the whole tile in VGPRs.
__device__ __forceinline__ void scale_acc(f32x16& acc, float c) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float x = acc[e], t;
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(t)
                 : "v"(c));
    acc[e] = x;
  }
}

// ---------------------------------------------------------------------------
// Cross-lane reductions inside a wave.
// ---------------------------------------------------------------------------
// max(x[l], x[l ^ 32]) for every lane, through v_permlane32_swap.
__device__ __forceinline__ float max_xor32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// max(x[l], x[l ^ 16]) within each half-wave, through v_permlane16_swap.
__device__ __forceinline__ float max_xor16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---------------------------------------------------------------------------
// 8x8 transpose of 16-bit elements held as 8 rows x 4 dwords.
// in[r] holds row r (elements 2j, 2j+1 in dword j); out[c] holds column c
// (rows 2j, 2j+1 in dword j).  Pure VALU byte permutes.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void transpose8x8_b16(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {      // dword j of every output = rows 2j, 2j+1
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) { // input dword c2 holds columns 2c2, 2c2+1
      uint32_t x = in[2 * j][c2];
      uint32_t y = in[2 * j + 1][c2];
      out[2 * c2][j] = __builtin_amdgcn_perm(y, x, 0x05040100u);      // lo halves
      out[2 * c2 + 1][j] = __builtin_amdgcn_perm(y, x, 0x07060302u);  // hi halves
    }
  }
}

// 4x8 (rows x cols) 16-bit transpose: in[r] (r<4) holds row r as 4 dwords;
// out[c] (c<8) receives column c as 2 dwords (rows 0,1 | rows 2,3).
__device__ __forceinline__ void transpose4x8_b16(const u32x4 in[4], u32x2 out[8]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) {
      uint32_t x = in[2 * j][c2];
      uint32_t y = in[2 * j + 1][c2];
      out[2 * c2][j] = __builtin_amdgcn_perm(y, x, 0x05040100u);
      out[2 * c2 + 1][j] = __builtin_amdgcn_perm(y, x, 0x07060302u);
    }
  }
}

// ---------------------------------------------------------------------------
// LDS helpers.
// ---------------------------------------------------------------------------
// ds_read_b64_tr_b16 (gfx950 transposing LDS read).  Within each group of
// 16 lanes, lane 4a+b receives element b of the 8-byte rows addressed by
// lanes a, 4+a, 8+a, 12+a (in that order).  Pointing lane 4j+a at
// V[key_j][d0 + 4a] therefore hands lane 4a+b the column d0+4a+b for keys
// key_0..key_3: a k-contiguous MFMA operand read straight from row-major V.
__device__ __forceinline__ u32x2 lds_read_tr16(const unsigned char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(__attribute__((address_space(3))) const unsigned char*)p);
  return __builtin_bit_cast(u32x2, r);
}

// LDS reads from a 32-bit LDS byte address (see lds_addr), for kernels
// that precompute lane addresses once: the compiler then folds the
// remaining compile-time offsets into the instruction's offset field.
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
__device__ __forceinline__ u32x4 lds_ld128(uint32_t addr) { return *(lds_u32x4*)(uintptr_t)addr; }
__device__ __forceinline__ u32x2 lds_read_tr16_at(uint32_t addr) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)addr));
}

// Running-sum helper: acc + x.lo + x.hi for a dword of two bf16 / f16.
template <typename T>
__device__ __forceinline__ float dot2_ones(uint32_t x, float acc);
template <>
__device__ __forceinline__ float dot2_ones<BF16>(uint32_t x, float acc) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, x), bf2{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
}
template <>
__device__ __forceinline__ float dot2_ones<F16>(uint32_t x, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x), h2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
}

// Direct global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4).
// Lane i reads 16 bytes at sbase + voff_i and they land at LDS byte address
// lds_addr + 16*i: one instruction fills 1 KB of LDS in lane order without
// passing through VGPRs.  sbase and lds_addr are wave-uniform (SGPRs).
//
// Issued as inline asm on purpose: the compiler then does not know that
// LDS is written behind its back, so it inserts none of its conservative
// vmcnt(0) waits before LDS reads.  The caller owns the synchronisation:
// wait_vmcnt<n>() until the loads of a stage have landed, then a barrier
// before other waves read them, and nothing of its own may be outstanding
// on vmcnt that the compiler would wait for with a smaller count (complete
// compiler-visible global loads with wait_vmcnt<0>() before issuing these).
// M0 is clobbered; no code here relies on M0 across the statement.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  // s_nop: one wait state between an SALU write of M0 and an LDS-DMA load.
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %0" ::"s"(sbase), "v"(voff), "s"(lds_addr)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier without the release/acquire fences of __syncthreads().
// Those fences make the compiler drain every outstanding LDS access of the
// wave (lgkmcnt(0)) before the barrier, which empties a read lookahead.  For
// kernels that order their LDS traffic themselves: DMA'd tiles are waited
// for with wait_vmcnt before the barrier, and a stage handed back to the DMA
// after the barrier was consumed by instructions that already waited for
// their reads.  The empty asm statements keep the compiler from moving
// memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Scheduling of one region of NM MFMAs and R LDS reads (issued in that
// region for a later use): alternate one MFMA with an even share of the
// reads, so a read lookahead never needs more than a few LDS instructions in
// flight (lgkmcnt counts at most 15) and the compiler can wait for exactly
// the reads each MFMA needs.  Call right after the region's code, before a
// sched_barrier that closes the region.
template <int NM, int R, int I = 0>
__device__ __forceinline__ void interleave_mfma_ds() {
  if constexpr (I < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    constexpr int r = (R * (I + 1)) / NM - (R * I) / NM;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);  // r LDS reads
    interleave_mfma_ds<NM, R, I + 1>();
  }
}

// Make the kernel-argument loads of `xs` complete here.  Arguments used
// only after a kernel's main loop (an output pointer) are otherwise loaded
// before the loop and left pending; the compiler then treats the lgkm
// counter as unordered at the loop head (scalar loads return out of order)
// and waits for every outstanding LDS read there (lgkmcnt(0)).
template <typename T>
__device__ __forceinline__ void land_arg(const T& x) {
  asm volatile("" ::"s"(x));
}
template <typename... Ts>
__device__ __forceinline__ void land_args(const Ts&... xs) {
  (land_arg(xs), ...);
}

// 32-bit LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) unsigned char*)p);
}

// s_waitcnt vmcnt(n) with the other counters untouched (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---------------------------------------------------------------------------
// Global memory helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st128(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ld64(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st64(void* p, const u32x2& v) { *reinterpret_cast<u32x2*>(p) = v; }

__device__ __forceinline__ u32x4 ld128_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st128_nt(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// XCD-aware block remap.  The dispatcher places workgroup i on XCD i % 8;
// renumbering so that consecutive logical tiles share an XCD keeps tiles
// that reuse the same operands inside one L2.  Valid for any nblocks: the
// tail that does not fill all 8 XCDs evenly keeps its identity mapping.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcd = 8;
  const int full = (nblocks / kXcd) * kXcd;
  if (bid >= full) return bid;
  const int per = full / kXcd;
  return (bid % kXcd) * per + bid / kXcd;
}

}  // namespace mx

// Host-side error plumbing shared by the entry points.
#define MX_RETURN_IF_HIP(expr)                   \
  do {                                           \
    hipError_t _e = (expr);                      \
    if (_e != hipSuccess) return MX_ERR_LAUNCH;  \
  } while (0)

namespace mx {

// Raise kernel F's dynamic-LDS limit to `bytes` once per device and
// process (thread-safe), instead of on every launch: the attribute call
// is host work that the few-microsecond decode launches would otherwise
// pay each time.  `bytes` is a constant of each kernel instantiation.
constexpr int kMaxDevices = 64;
template <auto F>
inline hipError_t lds_limit_once(int bytes) {
  static std::once_flag once[kMaxDevices];
  static hipError_t rc[kMaxDevices];
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices)
    return hipFuncSetAttribute((const void*)F, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  std::call_once(once[dev], [&] {
    rc[dev] = hipFuncSetAttribute((const void*)F, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  });
  return rc[dev];
}

}  // namespace mx
