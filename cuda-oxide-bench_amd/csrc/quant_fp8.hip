// fp8 (OCP e4m3) activation quantisation with 1x128 block scales, for gfx950.
//
// For every row m and 128-wide column block kb of X[M,K] (bf16 or f16):
//     s[m,kb] = amax_{k in kb} |X[m,k]| / 448        (1.0 for an all-zero block)
//     Q[m,k]  = e4m3(RNE(clamp(X[m,k] / s[m,kb], -448, 448)))
// so that X ~= Q * s.  This produces the A operand (and its sA scales) of
// mx_gemm_fp8_bs on the device: the activation side of the DeepSeek-V3
// style 1x128 / 128x128 block-scaled fp8 GEMM whose unscaled core is
// mojo-matmul-fp8/matmul_fp8.mojo:48-218.
//
// MI355X design (HBM-bound: 2 bytes in, 1 byte + 4/128 bytes out per value):
//  * one lane owns 16 consecutive values of a block (two 128-bit loads, one
//    128-bit store of 16 e4m3 bytes); 8 lanes cover a block, a wave 8
//    blocks, so every wave streams 2 KB of input in one pass;
//  * the block amax is a 3-step xor butterfly over the 8 lanes;
//  * X / s is the correctly rounded fp32 quotient, so the codes are
//    bit-identical to the host recipe.  A full IEEE division costs ~10 VALU
//    instructions; all 16 values of a lane share s, so the lane takes one
//    correctly rounded reciprocal r = RN(1/s) and refines per value:
//    q0 = RN(x r) (up to ~1.5 ulp off: r's half ulp plus the product's),
//    q1 = RN(q0 + (x - q0 s) r) (within one ulp), q2 = RN(q1 + (x - q1 s) r).
//    By Markstein's theorem (r correctly rounded, q1 within one ulp of x/s,
//    no underflow or overflow; the residual x - q1 s is then exact in one
//    FMA) q2 = RN(x/s); its sign is taken from x so that -0 stays -0.
//    Blocks with s outside [2^-90, 2^100] (tiny or
//    infinite amax) take the plain division, so every residual that can
//    reach a nonzero e4m3 code is a normal fp32 number;
//  * the packed converts (v_cvt_pk_fp8_f32, round to nearest even) do the
//    e4m3 encoding;
//  * non-finite inputs follow the host recipe: a block holding a NaN gets
//    scale 1, a block whose amax is infinite gets scale inf (its finite
//    values encode to +-0, its infinities to NaN), and NaN stays NaN.
#include "mx_common.h"

namespace mx {
namespace quant {

constexpr float kE4M3Max = 448.0f;
constexpr int NT = 256;               // 4 waves
constexpr int BPW = 8;                // blocks per wave
constexpr int BPG = BPW * NT / 64;    // blocks per workgroup

template <typename T>
__global__ __launch_bounds__(NT) void quant_fp8_act_kernel(const uint16_t* __restrict__ X, uint8_t* __restrict__ Q,
                                                          float* __restrict__ S, int M, int K, int ldx) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane & 7;  // 16-value slice of the block
  const int nkb = K / 128;
  const long long nblk = (long long)M * nkb;
  const long long gb = (long long)blockIdx.x * BPG + wave * BPW + (lane >> 3);
  const bool live = gb < nblk;
  const long long g = live ? gb : nblk - 1;  // dead lanes mirror the last block (never stored)
  const int row = (int)(g / nkb), kb = (int)(g % nkb);

  const uint16_t* src = X + (size_t)row * ldx + (size_t)kb * 128 + 16 * sub;
  const u32x4 a = ld128(src), b = ld128(src + 8);
  float v[16];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    v[2 * w] = T::to_f32(a[w] & 0xffffu);
    v[2 * w + 1] = T::to_f32(a[w] >> 16);
    v[8 + 2 * w] = T::to_f32(b[w] & 0xffffu);
    v[8 + 2 * w + 1] = T::to_f32(b[w] >> 16);
  }
  // Block amax; a NaN anywhere in the block makes its scale 1 (the host
  // recipe's amax is then NaN and `amax > 0` false).
  float amax = 0.f;
  int nan = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    amax = fmaxf(amax, fabsf(v[i]));
    nan |= v[i] != v[i];
  }
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off, 8));
    nan |= __shfl_xor(nan, off, 8);
  }
  const float s = nan ? 1.0f : (amax > 0.f ? amax / kE4M3Max : 1.0f);

  // y = clamp(x / s, -448, 448) with x / s correctly rounded: the
  // reciprocal refinement when every lane's block allows it (finite values,
  // s in range: the common case), else the plain division, which also
  // carries the non-finite cases (x / 1 in a block with a NaN; +-0 and
  // inf / inf = NaN in a block whose amax is infinite) with NaN kept NaN
  // through the clamp.
  float y[16];
  if (__all(!nan && s >= 0x1p-90f && s <= 0x1p100f)) {
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float q0 = v[i] * r;
      const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, s, v[i]), r, q0);
      // x = -0 would come out +0 (the residual is +0), where -0 / s is -0;
      // every other quotient already carries x's sign
      const float q = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q1, s, v[i]), r, q1), v[i]);
      y[i] = fminf(fmaxf(q, -kE4M3Max), kE4M3Max);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float q = v[i] / s;
      y[i] = q != q ? q : fminf(fmaxf(q, -kE4M3Max), kE4M3Max);
    }
  }

  u32x4 out;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    int p = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * w], y[4 * w + 1], 0, false);
    p = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * w + 2], y[4 * w + 3], p, true);
    out[w] = (uint32_t)p;
  }
  if (live) {
    st128(Q + (size_t)row * K + (size_t)kb * 128 + 16 * sub, out);
    if (sub == 0) S[(size_t)row * nkb + kb] = s;
  }
}

}  // namespace quant
}  // namespace mx

extern "C" int mx_quant_fp8_act(const void* X, void* Q, float* scales, int M, int K, int ldx, int dtype,
                                void* stream) {
  using namespace mx::quant;
  if (!X || !Q || !scales) return MX_ERR_NULL;
  if (M <= 0 || K <= 0 || ldx < K) return MX_ERR_SHAPE;
  if (K % 128) return MX_ERR_SHAPE;
  if (ldx % 8) return MX_ERR_ALIGN;
  if (((uintptr_t)X | (uintptr_t)Q) & 15) return MX_ERR_ALIGN;
  if ((uintptr_t)scales & 3) return MX_ERR_ALIGN;
  if (dtype != MX_DTYPE_BF16 && dtype != MX_DTYPE_F16) return MX_ERR_DTYPE;
  const long long nblk = (long long)M * (K / 128);
  const long long grid = (nblk + BPG - 1) / BPG;
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MX_DTYPE_BF16)
    hipLaunchKernelGGL(quant_fp8_act_kernel<mx::BF16>, dim3((unsigned)grid), dim3(NT), 0, s, (const uint16_t*)X,
                       (uint8_t*)Q, scales, M, K, ldx);
  else
    hipLaunchKernelGGL(quant_fp8_act_kernel<mx::F16>, dim3((unsigned)grid), dim3(NT), 0, s, (const uint16_t*)X,
                       (uint8_t*)Q, scales, M, K, ldx);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}
