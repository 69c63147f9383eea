// bf16 GEMM for gfx950:  C[M,N] = A[M,K] · B[K,N], fp32 accumulate, bf16 out.
//
// Semantics follow cutile-matmul-tc-bf16/main.py:59-78 (bf16 x bf16 -> f32
// accumulator -> bf16 store, zero padding at ragged edges) and the bf16 row
// of cutile-matmul-tiled-mixed/main.py:121-130.
//
// Design (MI355X-first, not a translation of the reference's cuTile/WMMA
// kernels):
//  * One workgroup computes a BM x BN tile of C with WM x WN waves; each
//    wave owns a (BM/WM) x (BN/WN) sub-tile built from 16x16x32 bf16 MFMAs.
//  * K advances in 64-deep tiles staged through LDS, double buffered: the
//    next tile's global loads are in flight while MFMAs consume the current
//    one, and one barrier per K tile separates the buffers.
//  * B is row-major (n contiguous) but the MFMA wants k-contiguous operand
//    registers, so each thread transposes an 8(k) x 8(n) (or 4x8) block of
//    B in registers with byte permutes before writing it to LDS as B^T.
//    Both LDS tiles are then k-contiguous and every operand fetch is one
//    ds_read_b128.
//  * LDS rows are 128 B (64 bf16); 16-byte chunks are XOR-swizzled with
//    (row ^ row>>3) & 7 so that fragment reads (16 consecutive rows, same
//    chunk) and the transposed B writes (rows 8 apart) are conflict-free.
//  * MFMAs are issued as D^T = B^T·A^T so each lane ends up holding four
//    consecutive n of one row of C: the epilogue writes 8-byte bf16 quads.
//  * Workgroup ids are remapped so that tiles sharing A rows / B columns
//    run on the same XCD (own L2), in groups of GROUP_M tile rows.
#include "mx_common.h"

namespace mx {
namespace gemm {

constexpr int BK = 64;        // K tile depth (bf16 elements)
constexpr int ROW_B = BK * 2; // bytes per LDS row
constexpr int GROUP_M = 8;

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// Byte offset of 16-byte chunk `c` (0..7) of LDS row `row`.
__device__ __forceinline__ int lds_off(int row, int c) { return row * ROW_B + ((c ^ swz(row)) << 4); }

template <int BM, int BN, int WM, int WN>
struct Cfg {
  static constexpr int NT = 64 * WM * WN;          // threads
  static constexpr int TM = BM / WM, TN = BN / WN; // wave tile
  static constexpr int FM = TM / 16, FN = TN / 16; // 16x16 fragments per wave
  static constexpr int A_CHUNKS = BM * BK / 8 / NT; // 16-B chunks of A per thread
  static constexpr int KR = BK * BN / 8 / NT;       // k rows per B block (x 8 n)
  static constexpr int B_BLOCKS_N = BN / 8;
  static constexpr int LDS_A = BM * ROW_B;
  static constexpr int LDS_B = BN * ROW_B;
  static constexpr int LDS_STAGE = LDS_A + LDS_B;
  static_assert(A_CHUNKS >= 1 && BM * BK / 8 % NT == 0, "A tile split");
  static_assert(KR == 8 || KR == 4 || KR == 2, "B block depth");
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile");
};

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C, int M,
    int N, int K, int lda, int ldb, int ldc) {
  using CF = Cfg<BM, BN, WM, WN>;
  constexpr int NT = CF::NT, FM = CF::FM, FN = CF::FN, KR = CF::KR;
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- tile coordinates: XCD-aware remap, then grouped row-major order ----
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int nblk = tiles_m * tiles_n;
  int id = xcd_remap(blockIdx.x, nblk);
  const int per_group = GROUP_M * tiles_n;
  const int group = id / per_group;
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (id % per_group) % gsz;
  const int tn = (id % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;

  // ---- per-thread global load assignments ----
  // A: chunk q = tid + i*NT -> row q/8, chunk q%8 (8 lanes cover one row).
  // B: block (kb, nb) = (tid / (BN/8), tid % (BN/8)); rows k = kb*KR + r,
  //    columns n = nb*8 .. nb*8+7.
  const int b_nb = tid % CF::B_BLOCKS_N;
  const int b_kb = tid / CF::B_BLOCKS_N;

  u32x4 ra[CF::A_CHUNKS];
  u32x4 rb[KR];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      const int row = q >> 3, c = q & 7;
      const int gm = m0 + row, gk = k0 + c * 8;
      ra[i] = (gm < M && gk < K) ? ld128(A + (size_t)gm * lda + gk) : u32x4{0, 0, 0, 0};
    }
    const int gn = n0 + b_nb * 8;
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      const int gk = k0 + b_kb * KR + r;
      rb[r] = (gk < K && gn < N) ? ld128(B + (size_t)gk * ldb + gn) : u32x4{0, 0, 0, 0};
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
    // Transpose the KR x 8 block to 8 columns of KR k-values.
    const int kbyte = b_kb * KR * 2;  // byte offset of this block's k range in a row
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int n = b_nb * 8 + c;
      uint32_t w[KR / 2];
#pragma unroll
      for (int j = 0; j < KR / 2; ++j) {
        const uint32_t x = rb[2 * j][c >> 1], y = rb[2 * j + 1][c >> 1];
        w[j] = (c & 1) ? __builtin_amdgcn_perm(y, x, 0x07060302u) : __builtin_amdgcn_perm(y, x, 0x05040100u);
      }
      const int chunk = kbyte >> 4, within = kbyte & 15;
      unsigned char* dst = sb + lds_off(n, chunk) + within;
      if constexpr (KR == 8) {
        *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
      } else if constexpr (KR == 4) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
      } else {
        *reinterpret_cast<uint32_t*>(dst) = w[0];
      }
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int a_row0 = wm * CF::TM + (lane & 15);
  const int b_row0 = wn * CF::TN + (lane & 15);
  const int kq = lane >> 4;  // which 8-wide k chunk of a 32-deep step

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile((kt + 1) * BK);
    const unsigned char* sa = smem + cur * CF::LDS_STAGE;
    const unsigned char* sb = sa + CF::LDS_A;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const int c = ks * 4 + kq;
      u32x4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const u32x4*>(sa + lds_off(a_row0 + i * 16, c));
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[j] = *reinterpret_cast<const u32x4*>(sb + lds_off(b_row0 + j * 16, c));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16<BF16>(bfr[j], af[i], acc[i][j]);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n .. n+3] for each fragment ----
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int gm = m0 + wm * CF::TM + i * 16 + (lane & 15);
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int gn = n0 + wn * CF::TN + j * 16 + 4 * (lane >> 4);
      if (gn < N) {
        u32x2 v{pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])};
        st64(C + (size_t)gm * ldc + gn, v);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
static int launch(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                  hipStream_t stream) {
  using CF = Cfg<BM, BN, WM, WN>;
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const size_t smem = 2 * CF::LDS_STAGE;
  auto kern = gemm_bf16_kernel<BM, BN, WM, WN>;
  MX_RETURN_IF_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(CF::NT), smem, stream, (const uint16_t*)A, (const uint16_t*)B,
                     (uint16_t*)C, M, N, K, lda, ldb, ldc);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

}  // namespace gemm
}  // namespace mx

extern "C" int mx_gemm_bf16(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb,
                            int ldc, void* stream) {
  if (!A || !B || !C) return MX_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0) return MX_ERR_SHAPE;
  if (lda < K || ldb < N || ldc < N) return MX_ERR_SHAPE;
  if ((K % 8) || (N % 8) || (lda % 8) || (ldb % 8) || (ldc % 8)) return MX_ERR_ALIGN;
  if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const long long tiles256 = (long long)((M + 255) / 256) * ((N + 255) / 256);
  const long long tiles128 = (long long)((M + 127) / 128) * ((N + 127) / 128);
  // Enough 256x256 tiles to cover the 256 CUs at least twice -> big tiles;
  // otherwise trade tile size for parallelism.
  if (tiles256 >= 512) return mx::gemm::launch<256, 256, 2, 4>(A, B, C, M, N, K, lda, ldb, ldc, s);
  if (tiles128 >= 256) return mx::gemm::launch<128, 128, 2, 2>(A, B, C, M, N, K, lda, ldb, ldc, s);
  return mx::gemm::launch<64, 64, 2, 2>(A, B, C, M, N, K, lda, ldb, ldc, s);
}
