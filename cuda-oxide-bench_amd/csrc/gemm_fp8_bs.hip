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
//  * The kernel computes C^T = B^T . A^T with 32x32x64 f8f6f4 MFMAs: the
//    B^T fragment (rows n) is the A operand, the A^T fragment (columns m)
//    the B operand.  A lane of the result then holds one m and 16 n, so the
//    1x128 activation scale is one per-lane value per fragment and the
//    128x128 weight scale one wave-uniform value.
//  * Each K tile is one 128-deep scale block: two MFMAs build a fresh fp32
//    partial per 32x32 fragment, promoted with one FMA per element,
//    acc += (sA[m,kb] * sB[kb,nb]) * partial (arbitrary fp32 scales, so the
//    power-of-two E8M0 hardware scales cannot carry them).  The fragments
//    of one row block build their partials side by side, so no MFMA waits
//    for the one just before it, and the promotion of one row block
//    overlaps the MFMAs of the next.
//  * 256x256 tiles, 8 waves (2 in m x 4 in n, two per SIMD), each wave
//    128(m) x 64(n): the fp32 accumulators stay in architectural VGPRs,
//    where the promotion FMAs can reach them.  Grids under 256 such tiles
//    use 128x128 tiles.
//  * A and B tiles go HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging) in their natural row-major layouts, double buffered.  A^T
//    fragments are plain ds_read_b128; B^T fragments come from k-major B
//    rows through gfx950's transposing read ds_read_b64_tr_b8: in each
//    16-lane group, lane 8h+b receives byte b of the 8-byte rows addressed
//    by lanes 2j+h, so pointing lane 2j+h at k-row j, columns 8h..8h+7
//    gives every lane 8 consecutive k-bytes of its own column.  No VALU
//    transposes.
//  * 16-byte chunks are XOR-swizzled per row so every fragment read phase
//    is bank-conflict free.
#include <type_traits>

#include "mx_common.h"

namespace mx {
namespace gemm8 {

constexpr int BK = 128;   // bytes of K per tile = one scale block
constexpr int NWAVES = 8;  // 2 (m) x 4 (n), two waves per SIMD
constexpr int NT = 64 * NWAVES;
constexpr int GROUP_M = 8;

// 32x32x64 e4m3 x e4m3 -> fp32 (scaled form with unit E8M0 scales).
// A: lane l holds row l%32, k = 32(l/32)..+31; B: column l%32, same k;
// D: lane l holds column l%32, rows 8i + 4(l/32) + j in d[4i + j].
__device__ __forceinline__ f32x16 mfma32_fp8(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__device__ __forceinline__ u32x2 lds_read_tr8_at(uint32_t addr) {
  typedef int v2i32 __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) v2i32 lds_v2i32;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i32*)(uintptr_t)addr));
}

template <int BM, int BN>
struct Cfg {
  static constexpr int WM = 2, WN = 4;
  static constexpr int TM = BM / WM, TN = BN / WN;   // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;   // 32x32 fragments
  static constexpr int A_B = BM * BK;                // A stage: BM rows of 128 B
  static constexpr int B_B = BK * BN;                // B stage: 128 k-rows of BN B
  static constexpr int STAGE = A_B + B_B;
  static constexpr int A_LPW = A_B / 1024 / NWAVES;  // 1 KB direct loads per wave
  static constexpr int B_LPW = B_B / 1024 / NWAVES;
  static constexpr int B_CH = BN / 16;               // 16-byte chunks per B row
  static constexpr int B_RPL = 1024 / BN;            // B rows per 1 KB load
  static_assert(FM >= 1 && FN >= 1 && A_LPW >= 1 && B_LPW >= 1, "tile split");
  static_assert(TN <= 128 && 128 % TN == 0, "a wave's columns share one weight-scale block");
  static_assert(BN == 128 || BN == 256, "B row swizzle");
};

// Chunk position swizzles.  A rows (128 B): a 16-lane b128 phase reads one
// chunk of 16 consecutive rows, two rows per 256 B.  B rows: a 32-lane
// transposing phase reads 8 consecutive k-rows x 2 adjacent chunks.
__device__ __forceinline__ int swz_a(int m) { return (m >> 1) & 7; }
template <int BN>
__device__ __forceinline__ int swz_b(int k) {
  return BN == 256 ? ((k & 7) << 1) : (((k >> 1) & 3) << 1);
}

template <int BM, int BN>
__global__ __launch_bounds__(NT, 1) void gemm_fp8_bs_kernel(const uint8_t* __restrict__ A,
                                                           const float* __restrict__ sA,
                                                           const uint8_t* __restrict__ B,
                                                           const float* __restrict__ sB,
                                                           uint16_t* __restrict__ C, int M, int N, int K) {
  using CF = Cfg<BM, BN>;
  constexpr int FM = CF::FM, FN = CF::FN;
  extern __shared__ __align__(1024) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / CF::WN, wn = wave % CF::WN;

  // ---- tile -> (tm, tn), grouped for L2 reuse, XCD-aware ----
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

  // ---- direct loads.  A load n: rows 8n .. 8n+7 (lane i: row 8n + i/8,
  // chunk (i%8) ^ swz_a(row)); B load n: k-rows B_RPL*n .. (lane i: k-row
  // B_RPL*n + i/B_CH, chunk (i%B_CH) ^ swz_b(row)).  Rows past M and
  // columns past N re-read the last valid ones (never stored). ----
  const uint32_t lds0 = lds_addr(smem);
  const bool full_m = m0 + BM <= M, full_n = n0 + BN <= N;
  uint32_t a_off[CF::A_LPW], b_off[CF::B_LPW];
#pragma unroll
  for (int n = 0; n < CF::A_LPW; ++n) {
    const int row = 8 * (wave * CF::A_LPW + n) + (lane >> 3);
    const int gm = full_m ? m0 + row : min(m0 + row, M - 1);
    a_off[n] = (uint32_t)(gm - m0) * K + 16 * ((lane & 7) ^ swz_a(row));
  }
#pragma unroll
  for (int n = 0; n < CF::B_LPW; ++n) {
    const int row = CF::B_RPL * (wave * CF::B_LPW + n) + lane / CF::B_CH;
    int col = 16 * ((lane % CF::B_CH) ^ swz_b<BN>(row));
    if (!full_n) col = min(n0 + col, N - 16) - n0;
    b_off[n] = (uint32_t)row * N + col;
  }
  // LDS layout [A0 | A1 | B0 | B1]: one base register per fragment reaches
  // both stages of its operand with the 16-bit immediate offset of ds_read.
  auto issue = [&](int kb, int stage) {
    const uint32_t sa = lds0 + stage * CF::A_B, sb = lds0 + 2 * CF::A_B + stage * CF::B_B;
    const uint8_t* abase = A + (size_t)m0 * K + (size_t)kb * BK;
    const uint8_t* bbase = B + (size_t)kb * BK * N + n0;
#pragma unroll
    for (int n = 0; n < CF::A_LPW; ++n) dma16(abase, a_off[n], sa + (wave * CF::A_LPW + n) * 1024);
#pragma unroll
    for (int n = 0; n < CF::B_LPW; ++n) dma16(bbase, b_off[n], sb + (wave * CF::B_LPW + n) * 1024);
  };

  // ---- fragment lane addresses (stage 0; stage 1 is an immediate away) ----
  // A^T (B operand): row m = wm*TM + 32 mf + l%32, chunks 4 ks + 2 (l/32) + {0,1}.
  const int am = wm * CF::TM + (lane & 31);
  const uint32_t a_row = lds0 + am * BK;
  const int a_x = swz_a(am);  // same for every mf (32 rows apart)
  // B^T (A operand) via tr_b8: in 16-lane group q, lane 2j+h reads k-row
  // 64 ks + 32 (q>>1) + 8 r + j, columns wn*TN + 32 nf + 16 (q&1) + 8 h.
  const int q = lane >> 4, jj = (lane & 15) >> 1, hh = lane & 1;
  const int b_k0 = 32 * (q >> 1) + jj;                       // plus 64 ks + 8 r
  const int b_c0 = wn * CF::TN + 16 * (q & 1) + 8 * hh;      // plus 32 nf
  const uint32_t b_row = lds0 + 2 * CF::A_B + b_k0 * BN;
  const int b_x = swz_b<BN>(b_k0);  // rows 8 apart share it
  uint32_t b_col[FN];
#pragma unroll
  for (int nf = 0; nf < FN; ++nf) {
    const int col = b_c0 + 32 * nf;
    b_col[nf] = b_row + 16 * ((col >> 4) ^ b_x) + (col & 15);
  }
  const int a_c = 2 * (lane >> 5);
  uint32_t a_col[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int h = 0; h < 2; ++h) a_col[ks][h] = a_row + 16 * ((4 * ks + a_c + h) ^ a_x);

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};

  // Block scales: sA row of this lane per m fragment, sB per wave.  The
  // scales of tile kb+1 are loaded before its tile loads are issued, so
  // the wait that lands the tile also lands them.
  int sa_row[FM];
#pragma unroll
  for (int mf = 0; mf < FM; ++mf) sa_row[mf] = min(m0 + am + 32 * mf, M - 1) * kblocks;
  const int wave_nb = min((n0 + wn * CF::TN) / 128, nblocks_n - 1);
  // The weight scale is wave-uniform, but it is loaded with a vector load
  // (an opaque per-lane zero offset): a scalar load would share lgkmcnt with
  // the LDS reads and return out of order, turning every LDS wait of the
  // tile into lgkmcnt(0).
  int vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  float sa_c[FM], sb_c;
  auto load_scales = [&](int kb) {
    sb_c = sB[(size_t)kb * nblocks_n + wave_nb + vzero];
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) sa_c[mf] = sA[sa_row[mf] + kb];
  };

  // One K tile (= one scale block) in stage STG.  Reads go out in the order
  // the MFMAs consume them; the A^T fragment of each k half is re-read for
  // the next row block right after its MFMAs are issued.  The fragments of
  // one row block build their partials side by side, so no MFMA waits for
  // the one just before it; each partial is promoted with one FMA per
  // element.
  auto tile = [&](int kb, auto stg_tag) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr uint32_t oa = STG * CF::A_B, ob = STG * CF::B_B;
    wait_vmcnt<0>();  // this wave's loads of tile kb and its scales landed
    lds_barrier();    // tile kb visible to all waves; the other stage is free
    float s_m[FM];
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) s_m[mf] = sa_c[mf] * sb_c;
    if (kb + 1 < kblocks) {
      load_scales(kb + 1);
      issue(kb + 1, STG ^ 1);
    }
    auto read_b = [&](int ks, int nf) {
      u32x2 v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = lds_read_tr8_at(b_col[nf] + ob + (64 * ks + 8 * r) * BN);
      return i32x8{(int)v[0][0], (int)v[0][1], (int)v[1][0], (int)v[1][1],
                   (int)v[2][0], (int)v[2][1], (int)v[3][0], (int)v[3][1]};
    };
    auto read_a = [&](int mf, int ks) {
      const uint32_t r = oa + 32 * mf * BK;
      const u32x4 lo = lds_ld128(a_col[ks][0] + r);
      const u32x4 hi = lds_ld128(a_col[ks][1] + r);
      return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    };
    i32x8 bf[2][FN], a[2];
    bf[0][0] = read_b(0, 0);
    a[0] = read_a(0, 0);
#pragma unroll
    for (int nf = 1; nf < FN; ++nf) bf[0][nf] = read_b(0, nf);
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) bf[1][nf] = read_b(1, nf);
    a[1] = read_a(0, 1);
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) {
      f32x16 p[FN];
#pragma unroll
      for (int nf = 0; nf < FN; ++nf) p[nf] = mfma32_fp8(bf[0][nf], a[0], f32x16{});
      if (mf + 1 < FM) a[0] = read_a(mf + 1, 0);
#pragma unroll
      for (int nf = 0; nf < FN; ++nf) p[nf] = mfma32_fp8(bf[1][nf], a[1], p[nf]);
      if (mf + 1 < FM) a[1] = read_a(mf + 1, 1);
#pragma unroll
      for (int nf = 0; nf < FN; ++nf) acc[nf][mf] += s_m[mf] * p[nf];
    }
  };

  load_scales(0);
  issue(0, 0);
  for (int kb = 0; kb < kblocks; kb += 2) {
    tile(kb, std::integral_constant<int, 0>{});
    if (kb + 1 < kblocks) tile(kb + 1, std::integral_constant<int, 1>{});
  }

  // ---- store C: lane holds m = m0 + am + 32 mf, n = n0 + wn*TN + 32 nf + 8 i + 4 (l/32) + j ----
#pragma unroll
  for (int mf = 0; mf < FM; ++mf) {
    const int gm = m0 + am + 32 * mf;
    if (gm >= M) continue;
    uint16_t* crow = C + (size_t)gm * N;
#pragma unroll
    for (int nf = 0; nf < FN; ++nf)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gn = n0 + wn * CF::TN + 32 * nf + 8 * i + 4 * (lane >> 5);
        if (gn < N) {
          const f32x16& a = acc[nf][mf];
          st64(crow + gn, u32x2{pack_bf16x2(a[4 * i], a[4 * i + 1]), pack_bf16x2(a[4 * i + 2], a[4 * i + 3])});
        }
      }
  }
}

template <int BM, int BN>
static int launch(const void* A, const float* sA, const void* B, const float* sB, void* C, int M, int N, int K,
                  hipStream_t stream) {
  using CF = Cfg<BM, BN>;
  const long long tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7fffffffLL) return MX_ERR_SHAPE;
  const size_t smem = 2 * CF::STAGE;
  constexpr auto kern = gemm_fp8_bs_kernel<BM, BN>;
  MX_RETURN_IF_HIP(lds_limit_once<kern>((int)smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(NT), smem, stream, (const uint8_t*)A, sA, (const uint8_t*)B,
                     sB, (uint16_t*)C, M, N, K);
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
  if ((long long)N * 256 > 0xffffffffLL || (long long)K * 256 > 0xffffffffLL) return MX_ERR_SHAPE;
  if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return MX_ERR_ALIGN;
  if (((uintptr_t)sA | (uintptr_t)sB) & 3) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const long long tiles256 = (long long)((M + 255) / 256) * ((N + 255) / 256);
  if (tiles256 >= 256) return mx::gemm8::launch<256, 256>(A, sA, B, sB, C, M, N, K, s);
  return mx::gemm8::launch<128, 128>(A, sA, B, sB, C, M, N, K, s);
}
