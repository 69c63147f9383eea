// bf16 GEMM for gfx950:  C[M,N] = A[M,K] · B[K,N], fp32 accumulate, bf16 out.
//
// Semantics follow cutile-matmul-tc-bf16/main.py:59-78 (bf16 x bf16 -> f32
// accumulator -> bf16 store, zero padding at ragged edges) and the bf16 row
// of cutile-matmul-tiled-mixed/main.py:121-130.
//
// Design (MI355X-first, not a translation of the reference's cuTile/WMMA
// kernels):
//  * 32x32x16 bf16 MFMAs (the shape that reaches the bf16 peak on gfx950;
//    16x16x32 runs at about half of it).  One workgroup computes a BM x BN
//    tile of C with WM x WN waves; each wave owns a (BM/WM) x (BN/WN)
//    sub-tile of 32x32 fragments.
//  * K advances in 64-deep tiles staged through LDS, double buffered: the
//    next tile's global loads are in flight while MFMAs consume the current
//    one; one barrier per K tile.
//  * A is stored k-contiguous ([BM][64]); B is stored exactly as it sits in
//    memory ([64][BN], n contiguous) and its k-contiguous MFMA operand is
//    read with gfx950's transposing LDS read (ds_read_b64_tr_b16), so no
//    thread ever transposes B in registers.
//  * LDS rows are padded (A: +16 B, B: +64 B) so that the 16-lane phases of
//    the A reads and the 32-lane phases of the transposing B reads hit
//    distinct banks, and every fragment address is base + immediate.
//  * MFMAs are issued as D^T = B^T·A^T, so each lane holds runs of four
//    consecutive n of one row of C: the epilogue writes 8-byte bf16 quads.
//  * Workgroup ids are remapped so that tiles sharing A rows / B columns
//    run on the same XCD (own L2), in groups of GROUP_M tile rows.
#include "mx_common.h"

namespace mx {
namespace gemm {

constexpr int BK = 64;  // K tile depth (bf16 elements)
constexpr int GROUP_M = 8;

template <int BM, int BN, int WM, int WN>
struct Cfg {
  static constexpr int NT = 64 * WM * WN;          // threads
  static constexpr int TM = BM / WM, TN = BN / WN; // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32; // 32x32 fragments per wave
  static constexpr int A_ROW = BK * 2 + 16;        // bytes per A row in LDS
  static constexpr int B_ROW = BN * 2 + 64;        // bytes per B row in LDS
  static constexpr int A_CHUNKS = BM * BK / 8 / NT;  // 16-B chunks of A per thread
  static constexpr int B_CHUNKS = BK * BN / 8 / NT;  // 16-B chunks of B per thread
  static constexpr int LDS_A = BM * A_ROW;
  static constexpr int LDS_B = BK * B_ROW;
  static constexpr int LDS_STAGE = LDS_A + LDS_B;
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile split");
  static_assert(BM * BK / 8 % NT == 0 && BK * BN / 8 % NT == 0, "tile split");
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile");
};

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C, int M,
    int N, int K, int lda, int ldb, int ldc) {
  using CF = Cfg<BM, BN, WM, WN>;
  constexpr int NT = CF::NT, FM = CF::FM, FN = CF::FN;
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int g = lane >> 5;

  // ---- tile coordinates: XCD-aware remap, then grouped row-major order ----
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int nblk = tiles_m * tiles_n;
  const int id = xcd_remap(blockIdx.x, nblk);
  const int per_group = GROUP_M * tiles_n;
  const int group = id / per_group;
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (id % per_group) % gsz;
  const int tn = (id % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);

  // ---- global -> register staging.  A: chunk q -> row q/8, chunk q%8.
  //      B: chunk q -> k row q/(BN/8), column chunk q%(BN/8). ----
  u32x4 ra[CF::A_CHUNKS], rb[CF::B_CHUNKS];
  constexpr int BCH = BN / 8;

  auto load_tile = [&](int k0) {
    const bool full = interior && (k0 + BK <= K);  // uniform
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      const int gm = m0 + (q >> 3), gk = k0 + (q & 7) * 8;
      if (full) {
        ra[i] = ld128(A + (size_t)gm * lda + gk);
      } else {
        const bool ok = gm < M && gk < K;
        const u32x4 x = ld128(A + (size_t)min(gm, M - 1) * lda + min(gk, K - 8));
        ra[i] = ok ? x : u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < CF::B_CHUNKS; ++i) {
      const int q = tid + i * NT;
      const int gk = k0 + q / BCH, gn = n0 + (q % BCH) * 8;
      if (full) {
        rb[i] = ld128(B + (size_t)gk * ldb + gn);
      } else {
        const bool ok = gk < K && gn < N;
        const u32x4 x = ld128(B + (size_t)min(gk, K - 1) * ldb + min(gn, N - 8));
        rb[i] = ok ? x : u32x4{0, 0, 0, 0};
      }
    }
  };

  auto store_tile = [&](int stage) {
    unsigned char* sa = smem + stage * CF::LDS_STAGE;
    unsigned char* sb = sa + CF::LDS_A;
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<u32x4*>(sa + (q >> 3) * CF::A_ROW + (q & 7) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < CF::B_CHUNKS; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<u32x4*>(sb + (q / BCH) * CF::B_ROW + (q % BCH) * 16) = rb[i];
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  // Fragment addressing (32x32x16, k = 16 per step, lane half g holds k 8g..8g+7):
  //  A operand: row wm*TM + 32i + lane%32, 16-B chunk 2ks + g.
  //  B^T operand via transposing reads: lane (g, sg, 4j+a) reads B row
  //  (k) 16ks + 8g + 4r + j at column wn*TN + 32jn + 16sg + 4a, r = 0, 1.
  const int a_off = (wm * CF::TM + (lane & 31)) * CF::A_ROW + g * 16;
  const int b_sg = (lane >> 4) & 1, b_j = (lane >> 2) & 3, b_a = lane & 3;
  const int b_off = (8 * g + b_j) * CF::B_ROW + (wn * CF::TN + 16 * b_sg + 4 * b_a) * 2;

  const int nk = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile((kt + 1) * BK);
    const unsigned char* sa = smem + cur * CF::LDS_STAGE;
    const unsigned char* sb = sa + CF::LDS_A;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      u32x4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const u32x4*>(sa + a_off + i * 32 * CF::A_ROW + ks * 32);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const unsigned char* p = sb + b_off + (16 * ks) * CF::B_ROW + j * 64;
        const u32x2 lo = lds_read_tr16(p);
        const u32x2 hi = lds_read_tr16(p + 4 * CF::B_ROW);
        bfr[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32<BF16>(bfr[j], af[i], acc[i][j]);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n .. n+3], m = row of lane, n = 8r + 4g ----
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int gm = m0 + wm * CF::TM + i * 32 + (lane & 31);
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gn = n0 + wn * CF::TN + j * 32 + 8 * r + 4 * g;
        if (gn < N) {
          const f32x16& a = acc[i][j];
          st64(C + (size_t)gm * ldc + gn,
               u32x2{pack_bf16x2(a[4 * r], a[4 * r + 1]), pack_bf16x2(a[4 * r + 2], a[4 * r + 3])});
        }
      }
  }
}

template <int BM, int BN, int WM, int WN>
static int launch(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                  hipStream_t stream) {
  using CF = Cfg<BM, BN, WM, WN>;
  const long long tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7fffffffLL) return MX_ERR_SHAPE;
  const size_t smem = 2 * CF::LDS_STAGE;
  auto kern = gemm_bf16_kernel<BM, BN, WM, WN>;
  MX_RETURN_IF_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(CF::NT), smem, stream, (const uint16_t*)A,
                     (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc);
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
