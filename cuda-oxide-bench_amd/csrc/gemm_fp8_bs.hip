// fp8 (OCP e4m3) GEMM with 1x128 / 128x128 block scaling, for gfx950.
//
//   C[m,n] = sum_kb sA[m,kb] * sB[kb, n/128] * sum_{k in kb} A[m,k] * B[k,n]
//
// The unscaled e4m3 x e4m3 -> f32 product is the semantics of
// mojo-matmul-fp8/matmul_fp8.mojo:48-218; the per-block dequantisation
// scales and the bf16 output are what this path specifies (DeepSeek-V3
// style 1x128 activation / 128x128 weight blocks).
//
// MI355X design:
//  * 16x16x128 f8f6f4 MFMA: one instruction consumes exactly one 128-deep
//    scale block, so each K tile (BK = 128) produces a fresh fp32 partial per
//    16x16 fragment which is promoted into the running accumulator with one
//    FMA per element:  acc += (sA[m,kb] * sB[kb,nb]) * partial.  The block
//    scales are arbitrary fp32, so the E8M0 (power-of-two) hardware scales
//    cannot carry them; software promotion keeps the result exact to fp32.
//  * Tiles, LDS double buffering, the in-register B transpose (here a
//    4(k) x 16(n) byte transpose with v_perm) and the XOR-swizzled 128-byte
//    LDS rows follow the bf16 kernel; every operand fetch is ds_read_b128.
//  * sB is uniform over a wave's n range (<= 128 columns, block aligned) and
//    is read once per K tile; sA is read per fragment row.
#include "mx_common.h"

namespace mx {
namespace gemm8 {

constexpr int BK = 128;   // bytes of K per tile = one scale block
constexpr int ROW_B = BK;
constexpr int GROUP_M = 8;

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lds_off(int row, int c) { return row * ROW_B + ((c ^ swz(row)) << 4); }

template <int BM, int BN, int WM, int WN>
struct Cfg {
  static constexpr int NT = 64 * WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int A_CHUNKS = BM * BK / 16 / NT;
  static constexpr int NB = BN / 16;                 // 16-column blocks of B
  static constexpr int KR = BK * BN / 16 / NT;       // k rows per B block
  static constexpr int LDS_A = BM * ROW_B;
  static constexpr int LDS_B = BN * ROW_B;
  static constexpr int LDS_STAGE = LDS_A + LDS_B;
  static_assert(KR == 4 || KR == 8, "4x16 byte transposes per thread");
  static_assert(A_CHUNKS >= 1, "A split");
  static_assert(128 % TN == 0, "wave n-range inside one scale block");
};

// 4 rows x 16 bytes -> 16 columns x 4 bytes (column c gets rows 0..3 at byte c).
__device__ __forceinline__ void transpose4x16_b8(const u32x4 in[4], uint32_t out[16]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = in[0][j], b = in[1][j], c = in[2][j], d = in[3][j];
    const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);
    const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);
    const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);
    const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);
    out[4 * j + 0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);
    out[4 * j + 1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);
    out[4 * j + 2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
    out[4 * j + 3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
  }
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_fp8_bs_kernel(const uint8_t* __restrict__ A,
                                                                  const float* __restrict__ sA,
                                                                  const uint8_t* __restrict__ B,
                                                                  const float* __restrict__ sB,
                                                                  uint16_t* __restrict__ C, int M, int N, int K) {
  using CF = Cfg<BM, BN, WM, WN>;
  constexpr int NT = CF::NT, FM = CF::FM, FN = CF::FN;
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int per_group = GROUP_M * tiles_n;
  const int group = id / per_group;
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (id % per_group) % gsz;
  const int tn = (id % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;

  const int kblocks = K / BK;
  const int nblocks_n = (N + 127) / 128;

  const int b_nb = tid % CF::NB, b_kb = tid / CF::NB;
  constexpr int KR = CF::KR;
  u32x4 ra[CF::A_CHUNKS], rb[KR];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      const int row = q >> 3, c = q & 7;
      const int gm = m0 + row;
      ra[i] = (gm < M) ? ld128(A + (size_t)gm * K + k0 + c * 16) : u32x4{0, 0, 0, 0};
    }
    const int gn = n0 + b_nb * 16;
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      const int gk = k0 + b_kb * KR + r;
      rb[r] = (gn < N) ? ld128(B + (size_t)gk * N + gn) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tile = [&](int stage) {
    unsigned char* sa = smem + stage * CF::LDS_STAGE;
    unsigned char* sb = sa + CF::LDS_A;
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<u32x4*>(sa + lds_off(q >> 3, q & 7)) = ra[i];
    }
    uint32_t cols[KR / 4][16];
#pragma unroll
    for (int h = 0; h < KR / 4; ++h) transpose4x16_b8(rb + 4 * h, cols[h]);
    const int kbyte = b_kb * KR;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int n = b_nb * 16 + c;
      unsigned char* dst = sb + lds_off(n, kbyte >> 4) + (kbyte & 15);
      if constexpr (KR == 8) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{cols[0][c], cols[1][c]};
      } else {
        *reinterpret_cast<uint32_t*>(dst) = cols[0][c];
      }
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Rows of C this lane accumulates (one per fragment row i) and the
  // wave's scale-block column.
  const int a_row0 = wm * CF::TM + (lane & 15);
  const int b_row0 = wn * CF::TN + (lane & 15);
  const int kq = lane >> 4;
  const int wave_nblk = min((n0 + wn * CF::TN) / 128, nblocks_n - 1);

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < kblocks; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < kblocks) load_tile((kt + 1) * BK);
    const float sb_k = sB[(size_t)kt * nblocks_n + wave_nblk];
    float sa_k[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int gm = m0 + a_row0 + i * 16;
      sa_k[i] = (gm < M) ? sA[(size_t)gm * kblocks + kt] * sb_k : 0.f;
    }
    const unsigned char* sa = smem + cur * CF::LDS_STAGE;
    const unsigned char* sb = sa + CF::LDS_A;
    i32x8 bfr[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int r = b_row0 + j * 16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(sb + lds_off(r, 2 * kq));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(sb + lds_off(r, 2 * kq + 1));
      bfr[j] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = a_row0 + i * 16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(sa + lds_off(r, 2 * kq));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(sa + lds_off(r, 2 * kq + 1));
      const i32x8 af{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const f32x4 p = mfma16_fp8(bfr[j], af, f32x4{0.f, 0.f, 0.f, 0.f});
        acc[i][j] += sa_k[i] * p;
      }
    }
    if (kt + 1 < kblocks) store_tile(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int gm = m0 + wm * CF::TM + i * 16 + (lane & 15);
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int gn = n0 + wn * CF::TN + j * 16 + 4 * (lane >> 4);
      if (gn < N) {
        st64(C + (size_t)gm * N + gn,
             u32x2{pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])});
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
static int launch(const void* A, const float* sA, const void* B, const float* sB, void* C, int M, int N, int K,
                  hipStream_t stream) {
  using CF = Cfg<BM, BN, WM, WN>;
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const size_t smem = 2 * CF::LDS_STAGE;
  auto kern = gemm_fp8_bs_kernel<BM, BN, WM, WN>;
  MX_RETURN_IF_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(CF::NT), smem, stream, (const uint8_t*)A, sA, (const uint8_t*)B, sB,
                     (uint16_t*)C, M, N, K);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

}  // namespace gemm8
}  // namespace mx

extern "C" int mx_gemm_fp8_bs(const void* A, const float* sA, const void* B, const float* sB, void* C, int M, int N,
                              int K, void* stream) {
  if (!A || !sA || !B || !sB || !C) return MX_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0) return MX_ERR_SHAPE;
  if (K % 128) return MX_ERR_SHAPE;
  if (N % 16) return MX_ERR_ALIGN;
  if ((long long)M * K > (1LL << 40) || (long long)K * N > (1LL << 40)) return MX_ERR_SHAPE;
  if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return MX_ERR_ALIGN;
  if (((uintptr_t)sA | (uintptr_t)sB) & 3) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  return mx::gemm8::launch<128, 128, 2, 2>(A, sA, B, sB, C, M, N, K, s);
}
