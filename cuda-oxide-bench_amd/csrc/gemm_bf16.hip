// bf16 GEMM for gfx950:  C[M,N] = A[M,K] · B[K,N], fp32 accumulate, bf16 out.
//
// Semantics follow cutile-matmul-tc-bf16/main.py:59-78 (bf16 x bf16 -> f32
// accumulator -> bf16 store, zero padding at ragged edges) and the bf16 row
// of cutile-matmul-tiled-mixed/main.py:121-130.
//
// The kernels (MI355X-first designs, not translations of the reference's
// cuTile/WMMA kernels) all compute D^T = B^T . A^T, so each lane holds runs
// of four consecutive n of one row of C and the epilogue writes 8-byte bf16
// quads; workgroup ids are remapped so that tiles sharing A rows / B
// columns run on the same XCD (own L2), in groups of GROUP_M tile rows.
//
// gemm_bf16_dma16_kernel (the large problems: at least one 256x256 tile
// per CU, K % 32 == 0; also 128x128 tiles when those are at least one per
// CU): 16x16x32 bf16 MFMAs, 8 waves of 128x64 (64x32 at 128x128 tiles),
// A/B tiles copied HBM -> LDS by direct loads into a 5-stage (6 at
// 128x128) ring, one barrier per K tile, the next K tile's fragments read
// during the current tile's MFMAs.  Details at the kernel.
// gemm_bf16_dma16s_kernel takes the 256x256 tiles when K % 64 == 0: the
// same MFMAs and schedule, with A in 64-deep blocks of whole 128-byte lines
// through a ring of its own beside the B ring.
//
// gemm_bf16_sdma_kernel (about one 64x64 tile per CU and a long K, e.g.
// 1024^3): two wave groups split K, each with its own direct-load ring.
//
// gemm_bf16_stream_kernel (K % 64 == 0; M <= 64 and N >= 256, or at most 64
// tiles of 64x64 and K >= 512): products too small to fill the CUs with
// tiles stream B through workgroups of 32 columns x 32 or 64 rows whose
// waves split K.
//
// gemm_bf16_smallm_kernel / gemm_bf16_smallm_sk_kernel (batched items with
// M <= 32): single-wave or K-split 4-wave workgroups over the whole K.
//
// gemm_bf16_kernel (everything else: small or ragged-K problems; 32x32x16
// bf16 MFMAs):
//  * One workgroup computes a BM x BN tile of C with WM x WN waves; each
//    wave owns a (BM/WM) x (BN/WN) sub-tile of 32x32 fragments.
//  * K advances in 64-deep tiles staged through LDS via registers, double
//    buffered: the next tile's global loads are in flight while MFMAs
//    consume the current one; one barrier per K tile.  The loads are
//    buffer loads: chunks past M, N or K get an out-of-range offset and
//    read as zero, so edge tiles and the K tail run the same branch-free
//    code as interior ones.
//  * A is stored k-contiguous ([BM][64]); B is stored exactly as it sits in
//    memory ([64][BN], n contiguous) and its k-contiguous MFMA operand is
//    read with gfx950's transposing LDS read (ds_read_b64_tr_b16), so no
//    thread ever transposes B in registers.
//  * LDS rows are padded (A: +16 B, B: +64 B) so that the 16-lane phases of
//    the A reads and the 32-lane phases of the transposing B reads hit
//    distinct banks, and every fragment address is base + immediate.
#include <type_traits>

#include "mx_common.h"

namespace mx {
namespace gemm {

// The direct-load 16x16x32 kernel: K depth of a ring stage (bf16 elements),
// ring stages and waves at 256x256 tiles, and stages and waves across N at
// 128x128 tiles (16 KB stages; 6 measured best of 4..9 at 2048^3).
constexpr int DMA_BK = 32;
constexpr int DMA_NS = 5, DMA_WM = 2, DMA_WN = 4;
constexpr int D128_NS = 6, D128_WN = 4;

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

// gridDim.y indexes a batch of independent products whose operands sit
// sA / sB / sC elements apart (0 and gridDim.y = 1 for a single GEMM).
// KS > 1 splits K inside the workgroup: KS groups of WM x WN waves, each
// with its own double buffer, take consecutive runs of K tiles of the same
// C tile, and their fp32 accumulators are summed through LDS at the end.
// For grids of about one tile per CU, where the serial K loop's load latency
// (not the MFMAs) sets the time, it runs KS loads in flight per CU.
// PF = 2 stages the global loads two K tiles ahead in two register sets
// (the LDS double buffer is unchanged), for the same latency-bound case.
// Buffer resource over [base, base + 2^31 - 16) for loads whose offsets
// stay below 2^31; an offset of kOobOffset is out of range and reads zero.
constexpr uint32_t kOobOffset = 0x7ffffff0u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)kOobOffset, 0x00020000);
}
__device__ __forceinline__ u32x4 buffer_ld128(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0);
}
// The register-staged kernel's in-range offsets (BM rows of A, BK k-rows of
// B from a tile's base) stay below that range: leading dimensions up to
// 4M (A, BM = 256) and 16M (B) elements.
template <int BM>
inline bool staged_strides_ok(int lda, int ldb) {
  return (long long)lda * 2 * BM < (long long)kOobOffset && (long long)ldb * 2 * BK < (long long)kOobOffset;
}

template <int BM, int BN, int WM, int WN, int KS = 1, int PF = 1>
__global__ __launch_bounds__(64 * WM * WN * KS, 1) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C, int M,
    int N, int K, int lda, int ldb, int ldc, long long sA, long long sB, long long sC) {
  using CF = Cfg<BM, BN, WM, WN>;
  constexpr int NT = CF::NT, FM = CF::FM, FN = CF::FN;
  extern __shared__ __align__(16) unsigned char smem_all[];
  A += (size_t)blockIdx.y * sA;
  B += (size_t)blockIdx.y * sB;
  C += (size_t)blockIdx.y * sC;

  const int grp = KS > 1 ? (int)threadIdx.x / NT : 0;  // K group
  unsigned char* const smem = smem_all + grp * 2 * CF::LDS_STAGE;
  const int tid = (int)threadIdx.x % NT;
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

  // ---- global -> register staging.  A: chunk q -> row q/8, chunk q%8.
  //      B: chunk q -> k row q/(BN/8), column chunk q%(BN/8). ----
  static_assert(PF == 1 || PF == 2, "one or two register sets");
  u32x4 ra[PF][CF::A_CHUNKS], rb[PF][CF::B_CHUNKS];
  constexpr int BCH = BN / 8;

  // Loads go through buffer resources based at the K tile: a chunk past M,
  // N or K gets an offset past the resource's range and reads as zero, so
  // every tile, edge or interior, K tail or not, runs the same branch-free
  // code (the host keeps lda * 2 * BM and ldb * 2 * BK below 2^31).
  auto load_tile = [&](int k0, auto set_tag) {
    constexpr int SET = decltype(set_tag)::value;
    const __amdgpu_buffer_rsrc_t rs_a = tile_rsrc(A + (size_t)m0 * lda + k0);
    const __amdgpu_buffer_rsrc_t rs_b = tile_rsrc(B + (size_t)k0 * ldb + n0);
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, c = (q & 7) * 8;
      const bool ok = m0 + r < M && k0 + c < K;
      ra[SET][i] = buffer_ld128(rs_a, ok ? (uint32_t)r * (uint32_t)lda * 2u + 2u * c : kOobOffset);
    }
#pragma unroll
    for (int i = 0; i < CF::B_CHUNKS; ++i) {
      const int q = tid + i * NT;
      const int r = q / BCH, c = (q % BCH) * 8;
      const bool ok = k0 + r < K && n0 + c < N;
      rb[SET][i] = buffer_ld128(rs_b, ok ? (uint32_t)r * (uint32_t)ldb * 2u + 2u * c : kOobOffset);
    }
  };

  auto store_tile = [&](int stage, auto set_tag) {
    constexpr int SET = decltype(set_tag)::value;
    unsigned char* sa = smem + stage * CF::LDS_STAGE;
    unsigned char* sb = sa + CF::LDS_A;
#pragma unroll
    for (int i = 0; i < CF::A_CHUNKS; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<u32x4*>(sa + (q >> 3) * CF::A_ROW + (q & 7) * 16) = ra[SET][i];
    }
#pragma unroll
    for (int i = 0; i < CF::B_CHUNKS; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<u32x4*>(sb + (q / BCH) * CF::B_ROW + (q % BCH) * 16) = rb[SET][i];
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

  // this group's K tiles: [kt0, kt0 + cnt); every group runs nkg loop trips
  // so the barriers match
  const int nk_all = (K + BK - 1) / BK;
  const int nkg = (nk_all + KS - 1) / KS;
  const int kt0 = grp * nkg;
  const int nk = max(0, min(nkg, nk_all - kt0));
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, PF - 1>;
  // MFMAs of the K tile in LDS stage `stage`
  auto compute = [&](int stage) {
    const unsigned char* sa = smem + stage * CF::LDS_STAGE;
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
  };

  if (nk > 0) {
    load_tile(kt0 * BK, S0{});
    store_tile(0, S0{});
  }
  if constexpr (PF == 2) {
    if (nk > 1) load_tile((kt0 + 1) * BK, S1{});
  }
  __syncthreads();

  if constexpr (PF == 2) {
    // Iteration it: register set it&1 (its tile already in LDS) takes tile
    // it+2; stage it&1 holds tile it; set (it+1)&1, loaded one iteration
    // earlier, goes to stage (it+1)&1, freed by the previous barrier.
    auto step = [&](int it, auto par) {
      constexpr int P = decltype(par)::value;
      if (it < nk) {
        if (it + 2 < nk) load_tile((kt0 + it + 2) * BK, std::integral_constant<int, P>{});
        compute(P);
        if (it + 1 < nk) store_tile(P ^ 1, std::integral_constant<int, P ^ 1>{});
      }
      __syncthreads();
    };
    for (int it = 0; it < nkg; it += 2) {
      step(it, S0{});
      if (it + 1 < nkg) step(it + 1, S1{});
    }
  } else {
    for (int it = 0; it < nkg; ++it) {
      const int cur = it & 1;
      if (it < nk) {
        if (it + 1 < nk) load_tile((kt0 + it + 1) * BK, S0{});
        compute(cur);
        if (it + 1 < nk) store_tile(cur ^ 1, S0{});
      }
      __syncthreads();
    }
  }

  if constexpr (KS > 1) {
    // Sum the groups' accumulators into group 0's (the loop's last barrier
    // freed every stage).  Element e of thread t of group g >= 1 sits at
    // float ((g-1)·E + e)·NT + t: consecutive threads, consecutive banks.
    constexpr int E = FM * FN * 16;
    static_assert((KS - 1) * E * NT * 4 <= KS * 2 * CF::LDS_STAGE, "the partial sums fit in the stages");
    float* red = reinterpret_cast<float*>(smem_all);
    if (grp > 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) red[((grp - 1) * E + (i * FN + j) * 16 + e) * NT + tid] = acc[i][j][e];
    }
    __syncthreads();
    if (grp > 0) return;  // no barrier follows
#pragma unroll
    for (int q = 1; q < KS; ++q)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += red[((q - 1) * E + (i * FN + j) * 16 + e) * NT + tid];
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

// A-row chunk swizzle of the small-M kernels' LDS rows: a 16-lane
// ds_read_b128 phase reads one chunk of 16 consecutive rows, and chunk ^
// swz_a(m) puts them in 16 distinct 16-byte slots of the 256-byte bank
// window (64-byte rows: (m >> 2) & 3; 128-byte rows: (m >> 1) & 7).
template <int BK>
__device__ __forceinline__ int swz_a(int m) {
  return BK == 64 ? ((m >> 1) & 7) : ((m >> 2) & 3);
}

// ---------------------------------------------------------------------------
// gemm_bf16_sdma_kernel: grids of about one 64x64 tile per CU with a long K
// (1024^3).  There the time is the latency of streaming each tile's 64 rows
// of A and 64 columns of B (256 KB per CU at 1024^3), not the MFMAs, so the
// loads go HBM -> LDS directly through a deep ring:
//  * 8 waves = 2 K groups x (2 x 2 waves of 32x32); group q takes the K
//    tiles q*nk .. q*nk + nk - 1, and the two groups' accumulators are
//    summed through LDS at the end;
//  * each group has a 5-slot ring of 64-deep K tiles (A: 64 rows x 128 B,
//    B: 64 k-rows x 128 B; both groups fill the 160 KB of LDS) with four
//    tiles (64 KB) in flight;
//  * 16-byte chunks are XOR-swizzled per row, chunk ^ ((m >> 1) & 7) for A
//    and chunk ^ (((k >> 1) & 1) << 2) for B: LDS serves a 128-bit read in
//    16-lane groups keyed by lane bit 5 and the parity of lane bits 2..4,
//    a transposing 64-bit read in 32-lane halves, and both fragment reads
//    below then touch distinct bank slots within every group.
// Shapes: M, N multiples of 64, K a multiple of 128.
// ---------------------------------------------------------------------------
struct SCfg {
  static constexpr int BM = 64, BN = 64, BK = 64, NSL = 5, KSG = 2;
  static constexpr int NW = 8, NWG = NW / KSG, NT = 64 * NW;  // waves, waves per group, threads
  static constexpr int RA = BK * 2, RB = BN * 2;              // LDS row bytes (128)
  static constexpr int A_B = BM * RA, B_B = BK * RB;          // 8 KB each
  static constexpr int STAGE = A_B + B_B;
  static constexpr int GRP = NSL * STAGE;                     // ring of one group
  static constexpr int LDS = KSG * GRP;
  static constexpr int A_LPW = A_B / 1024 / NWG, B_LPW = B_B / 1024 / NWG;  // 1 KB loads per wave per tile
  static constexpr int LPW = A_LPW + B_LPW;
  static constexpr int RPL = 1024 / RA;                       // rows per 1 KB load
  static_assert(LDS <= 160 * 1024 && (NSL - 2) * LPW < 64 && RA == RB, "ring");
};
__device__ __forceinline__ int swz_sa(int m) { return (m >> 1) & 7; }
__device__ __forceinline__ int swz_sb(int k) { return ((k >> 1) & 1) << 2; }

__global__ __launch_bounds__(SCfg::NT, 1) void gemm_bf16_sdma_kernel(const uint16_t* __restrict__ A,
                                                                    const uint16_t* __restrict__ B,
                                                                    uint16_t* __restrict__ C, int M, int N, int K,
                                                                    int lda, int ldb, int ldc) {
  using CF = SCfg;
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave / CF::NWG, wg = wave % CF::NWG;  // K group, wave within the group
  const int wm = wg / 2, wn = wg % 2;
  const int g = lane >> 5;

  // ---- tile -> (tm, tn), grouped for L2 reuse, XCD-aware ----
  const int tiles_m = M / CF::BM, tiles_n = N / CF::BN;
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int per_group = GROUP_M * tiles_n;
  const int first_m = (id / per_group) * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int m0 = (first_m + (id % per_group) % gsz) * CF::BM;
  const int n0 = ((id % per_group) / gsz) * CF::BN;
  const int nk = K / CF::BK / CF::KSG;  // K tiles per group
  const int kt0 = grp * nk;

  // ---- direct loads: load n of this wave fills rows (k-rows) RPL*(wg*LPW+n)
  // + lane/8 of the tile, lane taking the chunk stored at position lane%8 ----
  const uint32_t lds0 = lds_addr(smem) + grp * CF::GRP;
  uint32_t a_off[CF::A_LPW], b_off[CF::B_LPW];
#pragma unroll
  for (int n = 0; n < CF::A_LPW; ++n) {
    const int row = CF::RPL * (wg * CF::A_LPW + n) + lane / 8;
    a_off[n] = (uint32_t)row * (uint32_t)lda * 2u + 16u * ((lane % 8) ^ swz_sa(row));
  }
#pragma unroll
  for (int n = 0; n < CF::B_LPW; ++n) {
    const int row = CF::RPL * (wg * CF::B_LPW + n) + lane / 8;
    b_off[n] = (uint32_t)row * (uint32_t)ldb * 2u + 16u * ((lane % 8) ^ swz_sb(row));
  }
  auto issue = [&](int kt, int slot) {
    const uint32_t st = lds0 + slot * CF::STAGE;
    const uint16_t* abase = A + (size_t)m0 * lda + (size_t)(kt0 + kt) * CF::BK;
    const uint16_t* bbase = B + (size_t)(kt0 + kt) * CF::BK * ldb + n0;
#pragma unroll
    for (int n = 0; n < CF::A_LPW; ++n) dma16(abase, a_off[n], st + (wg * CF::A_LPW + n) * 1024);
#pragma unroll
    for (int n = 0; n < CF::B_LPW; ++n) dma16(bbase, b_off[n], st + CF::A_B + (wg * CF::B_LPW + n) * 1024);
  };

  // ---- fragment addresses in slot 0.  A^T (B operand): m = 32 wm +
  // lane%32, k-chunk 2 ks + g.  B^T (A operand) by transposing reads: lane
  // (g, sg, 4j+a) reads k-row 16 ks + 8 g + j (+4 for the upper half),
  // columns 32 wn + 16 sg + 4a .. +3. ----
  const int am = 32 * wm + (lane & 31);
  uint32_t a_frag[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) a_frag[ks] = lds0 + am * CF::RA + 16 * ((2 * ks + g) ^ swz_sa(am));
  const int b_sg = (lane >> 4) & 1, b_j = (lane >> 2) & 3, b_a = lane & 3;
  const uint32_t b_frag = lds0 + CF::A_B + (8 * g + b_j) * CF::RB +
                          16 * (((32 * wn + 16 * b_sg + 4 * b_a) >> 3) ^ swz_sb(b_j)) + 8 * (b_a & 1);

  f32x16 acc = f32x16{};
  auto compute = [&](int slot) {
    const uint32_t so = slot * CF::STAGE;
    u32x4 af[4], bf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      af[ks] = lds_ld128(a_frag[ks] + so);
      const u32x2 lo = lds_read_tr16_at(b_frag + so + 16 * ks * CF::RB);
      const u32x2 hi = lds_read_tr16_at(b_frag + so + (16 * ks + 4) * CF::RB);
      bf[ks] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma32<BF16>(bf[ks], af[ks], acc);
  };

  land_args(C);  // C is used only after the K loop
  // Tiles 0 .. NSL-2 in flight; every iteration issues one more (past the
  // end the last tile again, into slots nobody reads), so the wait is the
  // same in every iteration: tile kt has landed once at most NSL-2 tiles
  // issued after it are outstanding.
#pragma unroll
  for (int p = 0; p < CF::NSL - 1; ++p) issue(min(p, nk - 1), p);
  for (int kt = 0; kt < nk; ++kt) {
    wait_vmcnt<(CF::NSL - 2) * CF::LPW>();
    lds_barrier();  // tile kt visible to every wave; slot (kt-1) % NSL free
    issue(min(kt + CF::NSL - 1, nk - 1), (kt + CF::NSL - 1) % CF::NSL);
    compute(kt % CF::NSL);
  }
  wait_vmcnt<0>();  // no load lands after this point
  __syncthreads();  // ... and every fragment read is done: the LDS is free

  // ---- sum the two groups' accumulators (group 1 -> LDS -> group 0) ----
  float* red = reinterpret_cast<float*>(smem);
  const int tid = threadIdx.x % (64 * CF::NWG);
  if (grp == 1) {
#pragma unroll
    for (int e = 0; e < 16; ++e) red[e * 64 * CF::NWG + tid] = acc[e];
  }
  __syncthreads();
  if (grp == 1) return;  // no barrier follows
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] += red[e * 64 * CF::NWG + tid];

  // ---- epilogue: lane holds m = m0 + am, n = n0 + 32 wn + 8 i + 4 g + {0..3} ----
  uint16_t* crow = C + (size_t)(m0 + am) * ldc + n0 + 32 * wn + 4 * g;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    st64(crow + 8 * i, u32x2{pack_bf16x2(acc[4 * i], acc[4 * i + 1]), pack_bf16x2(acc[4 * i + 2], acc[4 * i + 3])});
}

static int launch_sdma(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                       hipStream_t stream) {
  const long long tiles = (long long)(M / SCfg::BM) * (N / SCfg::BN);
  if (tiles > 0x7fffffffLL) return MX_ERR_SHAPE;
  constexpr auto kern = gemm_bf16_sdma_kernel;
  MX_RETURN_IF_HIP(lds_limit_once<kern>(SCfg::LDS));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(SCfg::NT), SCfg::LDS, stream, (const uint16_t*)A,
                     (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

// ---------------------------------------------------------------------------
// gemm_bf16_dma16_kernel: the direct-load design above on 16x16x32 MFMAs.
// Under a sustained full-chip MFMA load the 16x16x32 shape delivers about
// 11% more bf16 throughput than 32x32x16 on MI355X (same FLOPs, less
// operand/accumulator traffic per FLOP, so less power at the same clock
// cap), which is what sets the large-GEMM rate.
//
//  * BM x BN tile (256x256, or 128x128 for mid-size problems), BK = 32 (one
//    16x16x32 k-step per K tile), WM x WN waves, each owning (BM/WM) x
//    (BN/WN) of C as 16x16 fragments.
//  * Operand layouts (16x16x32): the "A" operand holds 8 consecutive k of
//    row l%16 at k-group l/16; "B" the same for column l%16; D holds rows
//    4(l/16)..+3 of column l%16.  Issued as D^T = B^T . A^T: B^T fragments
//    come from the K-major B tile by transposing reads (lane (kg, j, a)
//    reads k-row 8kg + 4r + j, columns 4a..+3, r = 0, 1), A^T fragments are
//    one 16-byte read of an A row; each lane's D is four consecutive n of
//    one row of C (an 8-byte store).
//  * A rows are 64 B and a fragment read covers 16 rows x 4 chunks: chunk
//    kg ^ ((m >> 1) & 3) is the XOR that measured conflict-free on gfx950
//    (SQ_LDS_BANK_CONFLICT 0; the (m >> 2) and (m & 3) forms conflict).  B
//    rows are 512 B or 256 B (same banks every row): a 32-lane phase of transposing
//    reads covers 8 k-rows (two k-groups x 4) of 32 bytes each, and chunk
//    c ^ 2((k & 3) | ((k >> 3) & 1) << 2) gives the 8 rows distinct 32-byte
//    slots.  The DMA applies the same XOR on the global side.
//  * Ring of NS stages, one barrier per K tile (as above).  Tile kt+1's
//    fragments are read during step kt: B^T ones into the other half of a
//    parity double buffer at the step's start, each A^T one in place right
//    after the four MFMAs that consumed the previous tile's.
// ---------------------------------------------------------------------------
template <int NS, int WM, int WN, int BM_ = 256, int BN_ = 256>
struct D16Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = 32;
  static constexpr int NW = WM * WN, NT = 64 * NW;
  static constexpr int TM = BM / WM, TN = BN / WN;  // wave block
  static constexpr int FM = TM / 16, FN = TN / 16;  // 16x16 fragments
  static constexpr int RA = BK * 2, RB = BN * 2;    // LDS row bytes
  static constexpr int A_B = BM * RA, B_B = BK * RB;
  static constexpr int STAGE = A_B + B_B;
  static constexpr int A_LPW = A_B / 1024 / NW;  // 1 KB loads per wave per stage
  static constexpr int B_LPW = B_B / 1024 / NW;
  static constexpr int LPW = A_LPW + B_LPW;
  static constexpr int A_CH = RA / 16, A_RPL = 1024 / RA;  // chunks per A row, A rows per load
  static constexpr int B_CH = RB / 16, B_RPL = 1024 / RB;
  static_assert(NS >= 4 && NS <= 9 && NS * STAGE <= 160 * 1024, "LDS ring");
  static_assert((NS - 3) * LPW < 64, "vmcnt range");
  static_assert(A_LPW >= 1 && B_LPW >= 1 && FM >= 1 && FN >= 1, "tile split");
};
__device__ __forceinline__ int swz_a16(int m) { return (m >> 1) & 3; }
// Schedule of one K tile: per row block FN MFMAs, then LDS reads: the 2FN
// B^T reads spread over the first half of the row blocks, each A^T read
// right behind its row block.
template <int FM, int FN, int I = 0>
__device__ __forceinline__ void interleave_rows16() {
  if constexpr (I < FM) {
    constexpr int HB = FM / 2;
    constexpr int nb = I < HB ? (2 * FN * (I + 1)) / HB - (2 * FN * I) / HB : 0;
    __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1 + nb, 0);
    interleave_rows16<FM, FN, I + 1>();
  }
}
__device__ __forceinline__ int swz_b16(int k) { return 2 * ((k & 3) | (((k >> 3) & 1) << 2)); }

// Steps I .. P-1 of a period of the K loop: stage I % NS, parity I % 2.
template <int NS, int P, int I = 0, typename Step>
__device__ __forceinline__ void step_period(Step& step, int kt) {
  if constexpr (I < P) {
    step(kt + I, std::integral_constant<int, I % NS>{}, std::integral_constant<int, I % 2>{});
    step_period<NS, P, I + 1>(step, kt);
  }
}
// The first n (< P) steps of a period, for the tail of the K loop.
template <int NS, int P, int I = 0, typename Step>
__device__ __forceinline__ void step_tail(Step& step, int kt, int n) {
  if constexpr (I < P - 1) {
    if (I < n) {
      step(kt + I, std::integral_constant<int, I % NS>{}, std::integral_constant<int, I % 2>{});
      step_tail<NS, P, I + 1>(step, kt, n);
    }
  }
}

template <int NS, int WM, int WN, int BM_ = 256, int BN_ = 256>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_bf16_dma16_kernel(const uint16_t* __restrict__ A,
                                                                        const uint16_t* __restrict__ B,
                                                                        uint16_t* __restrict__ C, int M, int N,
                                                                        int K, int lda, int ldb, int ldc) {
  using CF = D16Cfg<NS, WM, WN, BM_, BN_>;
  constexpr int FM = CF::FM, FN = CF::FN, BK = CF::BK;
  extern __shared__ __align__(1024) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int kg = lane >> 4;  // k-group of the lane's operand and row quad of its result

  // ---- tile -> (tm, tn), grouped for L2 reuse, XCD-aware ----
  const int tiles_m = (M + CF::BM - 1) / CF::BM, tiles_n = (N + CF::BN - 1) / CF::BN;
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int per_group = GROUP_M * tiles_n;
  const int group = id / per_group;
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (id % per_group) % gsz;
  const int tn = (id % per_group) / gsz;
  const int m0 = tm * CF::BM, n0 = tn * CF::BN;
  const int nk = K / BK;

  // ---- direct-load lane offsets (bytes from the tile's first element).
  // Rows past M / columns past N re-read the last valid ones; their
  // results are never stored. ----
  const uint32_t lds0 = lds_addr(smem);
  const bool full_m = m0 + CF::BM <= M, full_n = n0 + CF::BN <= N;
  uint32_t a_off[CF::A_LPW], b_off[CF::B_LPW];
#pragma unroll
  for (int n = 0; n < CF::A_LPW; ++n) {
    const int row = CF::A_RPL * (wave * CF::A_LPW + n) + lane / CF::A_CH;
    const int gm = full_m ? m0 + row : min(m0 + row, M - 1);
    a_off[n] = (uint32_t)(gm - m0) * (uint32_t)lda * 2u + 16u * ((lane % CF::A_CH) ^ swz_a16(row));
  }
#pragma unroll
  for (int n = 0; n < CF::B_LPW; ++n) {
    const int row = CF::B_RPL * (wave * CF::B_LPW + n) + lane / CF::B_CH;
    int col = 8 * ((lane % CF::B_CH) ^ swz_b16(row));  // elements
    if (!full_n) col = min(n0 + col, N - 8) - n0;
    b_off[n] = (uint32_t)row * (uint32_t)ldb * 2u + 2u * col;
  }
  auto issue = [&](int kt, int stage) {
    const uint32_t st = lds0 + stage * CF::STAGE;
    const uint16_t* abase = A + (size_t)m0 * lda + (size_t)kt * BK;
    const uint16_t* bbase = B + (size_t)kt * BK * ldb + n0;
#pragma unroll
    for (int n = 0; n < CF::A_LPW; ++n) dma16(abase, a_off[n], st + (wave * CF::A_LPW + n) * 1024);
#pragma unroll
    for (int n = 0; n < CF::B_LPW; ++n) dma16(bbase, b_off[n], st + CF::A_B + (wave * CF::B_LPW + n) * 1024);
  };

  // ---- fragment lane addresses, one base per ring stage (stages lie past
  // ds_read's 16-bit immediate), fragments at immediates from it ----
  // A^T (B operand): row am + 16 mf, chunk kg ^ swz(am) (swz is the same
  // for every mf).
  const int am = wm * CF::TM + (lane & 15);
  uint32_t a_col[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    a_col[st] = lds0 + st * CF::STAGE + am * CF::RA + 16 * (kg ^ swz_a16(am));
    asm volatile("" : "+v"(a_col[st]));  // keep it a base register
  }
  // B^T (A operand): lane (kg, j, a) reads k-rows 8kg + 4r + j, columns
  // wn*TN + 16 nf + 4a .. +3 (8 bytes of a 16-byte chunk).
  const int b_j = (lane >> 2) & 3, b_a = lane & 3;
  const int bk = 8 * kg + b_j;  // k-row of the r = 0 read; r = 1 is 4 rows further, same swizzle
  uint32_t b_col[NS][FN];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) {
      const int chunk = (wn * CF::TN + 16 * nf + 4 * b_a) >> 3;
      b_col[st][nf] = lds0 + st * CF::STAGE + CF::A_B + bk * CF::RB + 16 * (chunk ^ swz_b16(bk)) + 8 * (b_a & 1);
      asm volatile("" : "+v"(b_col[st][nf]));
    }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{};

  u32x4 af[FM];     // A^T fragments of the current tile, refilled in place
  u32x4 bf[2][FN];  // B^T fragments, double buffered by tile parity
  auto read_b = [&](int stg, int buf) {
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) {
      const u32x2 lo = lds_read_tr16_at(b_col[stg][nf]);
      const u32x2 hi = lds_read_tr16_at(b_col[stg][nf] + 4 * CF::RB);
      bf[buf][nf] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };
  auto read_a = [&](int stg, int mf) { af[mf] = lds_ld128(a_col[stg] + 16 * mf * CF::RA); };

  // One K tile: its fragments are in af and bf[PAR].  Every step issues
  // exactly one tile of loads (near the end the last tile again, into
  // stages nobody reads), so the ring accounting is the same in every step.
  auto step = [&](int kt, auto stg_tag, auto par_tag) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr int PAR = decltype(par_tag)::value;
    constexpr int NXT = (STG + 1) % NS;
    // Every wave has read tile kt (during step kt-1) and its own loads of
    // tile kt+1 have landed (at most the NS-3 tiles issued after it are in
    // flight): after the barrier tile kt+1 is readable and stage
    // (kt-1)%NS, last read during step kt-2, takes tile kt+NS-1.
    wait_vmcnt<(NS - 3) * CF::LPW>();
    lds_barrier();
    issue(min(kt + NS - 1, nk - 1), (STG + NS - 1) % NS);
    __builtin_amdgcn_sched_barrier(0);
    read_b(NXT, PAR ^ 1);
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) {
#pragma unroll
      for (int nf = 0; nf < FN; ++nf) acc[mf][nf] = mfma16<BF16>(bf[PAR][nf], af[mf], acc[mf][nf]);
      read_a(NXT, mf);
    }
    interleave_rows16<FM, FN>();
    __builtin_amdgcn_sched_barrier(0);
  };

  land_args(C);  // C is used only after the K loop
  // Prologue: tiles 0 .. NS-2 in flight (tiles past the end re-load the
  // last one), wait for tile 0, read its fragments.
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) issue(min(p, nk - 1), p);
  wait_vmcnt<(NS - 2) * CF::LPW>();
  lds_barrier();
  read_b(0, 0);
#pragma unroll
  for (int mf = 0; mf < FM; ++mf) read_a(0, mf);
  // stage kt % NS and parity kt % 2 repeat every P tiles
  constexpr int P = NS % 2 == 0 ? NS : 2 * NS;
  int kt = 0;
  for (; kt + P <= nk; kt += P) step_period<NS, P>(step, kt);
  step_tail<NS, P>(step, kt, nk - kt);
  wait_vmcnt<0>();  // no DMA may land in LDS after the workgroup ends

  // ---- epilogue: lane holds m = am + 16 mf, n = wn*TN + 16 nf + 4 kg + {0..3}
  // of the tile.  The tile goes through LDS (bf16 rows padded by 16 bytes)
  // and is stored as whole rows, each lane 16 contiguous bytes, instead of
  // 8-byte pieces that the memory system writes back as partial lines.  The
  // ring is free once every wave is past its last fragment reads. ----
  constexpr int CROW = CF::BN * 2 + 16;
  static_assert(CF::BM * CROW <= NS * CF::STAGE, "C tile fits the ring");
  __syncthreads();
#pragma unroll
  for (int mf = 0; mf < FM; ++mf) {
    const int r = am + 16 * mf;
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) {
      const int c = wn * CF::TN + 16 * nf + 4 * kg;
      const f32x4& a = acc[mf][nf];
      *reinterpret_cast<u32x2*>(smem + r * CROW + 2 * c) = u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
    }
  }
  __syncthreads();
  {
    constexpr int CPR = CF::BN / 8;     // 16-byte chunks per tile row
    constexpr int RPI = CF::NT / CPR;   // rows per workgroup-wide store
    const int t = threadIdx.x;
    const int cc = t % CPR, r0 = t / CPR;
    const int gn = n0 + 8 * cc;
#pragma unroll 4
    for (int r = r0; r < CF::BM; r += RPI) {
      const int gm = m0 + r;
      if (gm < M && gn < N)
        st128(C + (size_t)gm * ldc + gn, *reinterpret_cast<const u32x4*>(smem + r * CROW + 16 * cc));
    }
  }
}

// ---------------------------------------------------------------------------
// gemm_bf16_dma16s_kernel: gemm_bf16_dma16_kernel's 256x256 tiles and
// fragment schedule with whole 128-byte A lines.  In the single ring, a
// 32-deep stage holds 64 bytes of each A row, so every A line is fetched as
// two half-line requests; the L1 then holds up the address unit (the fp8
// GEMM measured the same).  Here A goes through its own ring of 64-deep
// blocks (256 rows x 128 B, 3 slots) beside a ring of 32-deep B stages
// (32 k-rows x 512 B, 4 slots), 160 KB in all:
//  * step kt computes K tile kt (B stage kt, half kt % 2 of A block kt / 2)
//    and reads tile kt+1's fragments; it issues B stage kt+3 and half kt % 2
//    of A block kt/2 + 2, each into the slot of the stage / block that the
//    barrier just freed, so every step issues the same 4 loads per wave and
//    waits for all but the 4 of the step before.
//  * A rows of 8 chunks: chunk c ^ ((m >> 1) & 7) keeps the 16-lane phases
//    of the A^T reads on distinct bank slots.
// Shapes: K % 64 == 0 (whole A blocks).
// ---------------------------------------------------------------------------
struct S16Cfg {
  static constexpr int BM = 256, BN = 256, BK = 32, BKA = 64;
  static constexpr int WM = DMA_WM, WN = DMA_WN, NW = WM * WN, NT = 64 * NW;
  static constexpr int TM = BM / WM, TN = BN / WN;   // wave block
  static constexpr int FM = TM / 16, FN = TN / 16;   // 16x16 fragments
  static constexpr int RA = BKA * 2, RB = BN * 2;    // LDS row bytes (A 128, B 512)
  static constexpr int A_B = BM * RA, B_B = BK * RB;  // A block 32 KB, B stage 16 KB
  static constexpr int NSA = 3, NSB = 4;
  static constexpr int B_OFF = NSA * A_B;
  static constexpr int LDS = NSA * A_B + NSB * B_B;
  static constexpr int A_LPW = A_B / 1024 / NW;      // 1 KB loads per wave per A block
  static constexpr int B_LPW = B_B / 1024 / NW;      // ... per B stage
  static constexpr int A_RPL = 1024 / RA;            // A rows per load
  static constexpr int B_CH = RB / 16, B_RPL = 1024 / RB;
  static constexpr int VM = B_LPW + A_LPW / 2;       // loads per step and wave
  static constexpr int P = 12;                        // steps until slots and parity repeat
  static_assert(LDS <= 160 * 1024 && A_LPW % 2 == 0 && A_LPW >= 2 && B_LPW >= 1, "rings");
};
__device__ __forceinline__ int swz_a16w(int m) { return (m >> 1) & 7; }

template <int P, int I = 0, typename Step>
__device__ __forceinline__ void steps_s(Step& step, int kt) {
  if constexpr (I < P) {
    step(kt + I, std::integral_constant<int, I>{});
    steps_s<P, I + 1>(step, kt);
  }
}
template <int P, int I = 0, typename Step>
__device__ __forceinline__ void steps_tail_s(Step& step, int kt, int n) {
  if constexpr (I < P - 1) {
    if (I < n) {
      step(kt + I, std::integral_constant<int, I>{});
      steps_tail_s<P, I + 1>(step, kt, n);
    }
  }
}

__global__ __launch_bounds__(S16Cfg::NT, 1) void gemm_bf16_dma16s_kernel(const uint16_t* __restrict__ A,
                                                                        const uint16_t* __restrict__ B,
                                                                        uint16_t* __restrict__ C, int M, int N,
                                                                        int K, int lda, int ldb, int ldc) {
  using CF = S16Cfg;
  constexpr int FM = CF::FM, FN = CF::FN, BK = CF::BK, WN = CF::WN;
  extern __shared__ __align__(1024) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int kg = lane >> 4;  // k-group of the lane's operand and row quad of its result

  // ---- tile -> (tm, tn), grouped for L2 reuse, XCD-aware ----
  const int tiles_m = (M + CF::BM - 1) / CF::BM, tiles_n = (N + CF::BN - 1) / CF::BN;
  const int id = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int per_group = GROUP_M * tiles_n;
  const int group = id / per_group;
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (id % per_group) % gsz;
  const int tn = (id % per_group) / gsz;
  const int m0 = tm * CF::BM, n0 = tn * CF::BN;
  const int nk = K / BK, nka = K / CF::BKA;

  // ---- direct-load lane offsets (bytes from the tile's first element).
  // Rows past M / columns past N re-read the last valid ones; their
  // results are never stored. ----
  const uint32_t lds0 = lds_addr(smem);
  const bool full_m = m0 + CF::BM <= M, full_n = n0 + CF::BN <= N;
  uint32_t a_off[CF::A_LPW], b_off[CF::B_LPW];
#pragma unroll
  for (int n = 0; n < CF::A_LPW; ++n) {
    const int row = CF::A_RPL * (wave * CF::A_LPW + n) + lane / 8;
    const int gm = full_m ? m0 + row : min(m0 + row, M - 1);
    a_off[n] = (uint32_t)(gm - m0) * (uint32_t)lda * 2u + 16u * ((lane % 8) ^ swz_a16w(row));
  }
#pragma unroll
  for (int n = 0; n < CF::B_LPW; ++n) {
    const int row = CF::B_RPL * (wave * CF::B_LPW + n) + lane / CF::B_CH;
    int col = 8 * ((lane % CF::B_CH) ^ swz_b16(row));  // elements
    if (!full_n) col = min(n0 + col, N - 8) - n0;
    b_off[n] = (uint32_t)row * (uint32_t)ldb * 2u + 2u * col;
  }
  // B stage s into B slot s % NSB; half h of A block j into A slot j % NSA.
  // Stages and blocks past the end re-load the last one (into slots no
  // later step reads).
  auto issue_b = [&](int s, int slot) {
    const uint16_t* bbase = B + (size_t)min(s, nk - 1) * BK * ldb + n0;
#pragma unroll
    for (int n = 0; n < CF::B_LPW; ++n)
      dma16(bbase, b_off[n], lds0 + CF::B_OFF + slot * CF::B_B + (wave * CF::B_LPW + n) * 1024);
  };
  auto issue_a = [&](int j, int h, int slot) {
    const uint16_t* abase = A + (size_t)m0 * lda + (size_t)min(j, nka - 1) * CF::BKA;
#pragma unroll
    for (int n = h * CF::A_LPW / 2; n < (h + 1) * CF::A_LPW / 2; ++n)
      dma16(abase, a_off[n], lds0 + slot * CF::A_B + (wave * CF::A_LPW + n) * 1024);
  };

  // ---- fragment lane addresses: one base per A slot and K half, and per
  // B slot and column fragment (slots lie past ds_read's 16-bit immediate) ----
  // A^T (B operand): row am + 16 mf, chunk (4 h + kg) ^ swz(am) (swz is the
  // same for every mf, 16 rows apart).
  const int am = wm * CF::TM + (lane & 15);
  uint32_t a_col[CF::NSA][2];
#pragma unroll
  for (int st = 0; st < CF::NSA; ++st)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      a_col[st][h] = lds0 + st * CF::A_B + am * CF::RA + 16 * ((4 * h + kg) ^ swz_a16w(am));
      asm volatile("" : "+v"(a_col[st][h]));  // keep it a base register
    }
  // B^T (A operand): lane (kg, j, a) reads k-rows 8kg + 4r + j, columns
  // wn*TN + 16 nf + 4a .. +3 (8 bytes of a 16-byte chunk).
  const int b_j = (lane >> 2) & 3, b_a = lane & 3;
  const int bk = 8 * kg + b_j;
  uint32_t b_col[CF::NSB][FN];
#pragma unroll
  for (int st = 0; st < CF::NSB; ++st)
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) {
      const int chunk = (wn * CF::TN + 16 * nf + 4 * b_a) >> 3;
      b_col[st][nf] = lds0 + CF::B_OFF + st * CF::B_B + bk * CF::RB + 16 * (chunk ^ swz_b16(bk)) + 8 * (b_a & 1);
      asm volatile("" : "+v"(b_col[st][nf]));
    }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{};

  u32x4 af[FM];     // A^T fragments of the current tile, refilled in place
  u32x4 bf[2][FN];  // B^T fragments, double buffered by tile parity
  auto read_b = [&](int stg, int buf) {
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) {
      const u32x2 lo = lds_read_tr16_at(b_col[stg][nf]);
      const u32x2 hi = lds_read_tr16_at(b_col[stg][nf] + 4 * CF::RB);
      bf[buf][nf] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };
  auto read_a = [&](int stg, int h, int mf) { af[mf] = lds_ld128(a_col[stg][h] + 16 * mf * CF::RA); };

  // Step kt = 12q + I: tile kt's fragments are in af and bf[I % 2]; B
  // stage kt sits in slot I % 4 and A block kt / 2 in slot (I / 2) % 3.
  auto step = [&](int kt, auto i_tag) {
    constexpr int I = decltype(i_tag)::value;
    constexpr int PAR = I % 2;
    constexpr int NB = (I + 1) % CF::NSB, NA = ((I + 1) / 2) % CF::NSA, NH = (I + 1) % 2;
    // Every wave has read tile kt (during step kt-1) and its own loads up
    // to those of step kt-2 have landed, tile kt+1's among them: after the
    // barrier tile kt+1 is readable, and B stage kt-1 (read during step
    // kt-2) and A block kt/2 - 1 (its last tile read no later) are free.
    wait_vmcnt<CF::VM>();
    lds_barrier();
    issue_b(kt + 3, (I + 3) % CF::NSB);
    issue_a(kt / 2 + 2, I % 2, (I / 2 + 2) % CF::NSA);
    __builtin_amdgcn_sched_barrier(0);
    read_b(NB, PAR ^ 1);
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) {
#pragma unroll
      for (int nf = 0; nf < FN; ++nf) acc[mf][nf] = mfma16<BF16>(bf[PAR][nf], af[mf], acc[mf][nf]);
      read_a(NA, NH, mf);
    }
    interleave_rows16<FM, FN>();
    __builtin_amdgcn_sched_barrier(0);
  };

  land_args(C);  // C is used only after the K loop
  // Prologue, in the order the waits need: A block 0, B stages 0 and 1,
  // A block 1, B stage 2; then tile 0's fragments.
  issue_a(0, 0, 0);
  issue_a(0, 1, 0);
  issue_b(0, 0);
  issue_b(1, 1);
  issue_a(1, 0, 1);
  issue_a(1, 1, 1);
  issue_b(2, 2);
  wait_vmcnt<2 * CF::B_LPW + CF::A_LPW>();  // B stage 1, A block 1 and B stage 2 may be in flight
  lds_barrier();
  read_b(0, 0);
#pragma unroll
  for (int mf = 0; mf < FM; ++mf) read_a(0, 0, mf);
  int kt = 0;
  for (; kt + CF::P <= nk; kt += CF::P) steps_s<CF::P>(step, kt);
  steps_tail_s<CF::P>(step, kt, nk - kt);
  wait_vmcnt<0>();  // no DMA may land in LDS after the workgroup ends

  // ---- epilogue (as gemm_bf16_dma16_kernel): the tile goes through LDS as
  // bf16 rows padded by 16 bytes and is stored as whole rows. ----
  constexpr int CROW = CF::BN * 2 + 16;
  static_assert(CF::BM * CROW <= CF::LDS, "C tile fits the rings");
  __syncthreads();
#pragma unroll
  for (int mf = 0; mf < FM; ++mf) {
    const int r = am + 16 * mf;
#pragma unroll
    for (int nf = 0; nf < FN; ++nf) {
      const int c = wn * CF::TN + 16 * nf + 4 * kg;
      const f32x4& a = acc[mf][nf];
      *reinterpret_cast<u32x2*>(smem + r * CROW + 2 * c) = u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
    }
  }
  __syncthreads();
  {
    constexpr int CPR = CF::BN / 8;     // 16-byte chunks per tile row
    constexpr int RPI = CF::NT / CPR;   // rows per workgroup-wide store
    const int t = threadIdx.x;
    const int cc = t % CPR, r0 = t / CPR;
    const int gn = n0 + 8 * cc;
#pragma unroll 4
    for (int r = r0; r < CF::BM; r += RPI) {
      const int gm = m0 + r;
      if (gm < M && gn < N)
        st128(C + (size_t)gm * ldc + gn, *reinterpret_cast<const u32x4*>(smem + r * CROW + 16 * cc));
    }
  }
}

static int launch_dma16s(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                         hipStream_t stream) {
  using CF = S16Cfg;
  const long long tiles = (long long)((M + CF::BM - 1) / CF::BM) * ((N + CF::BN - 1) / CF::BN);
  if (tiles > 0x7fffffffLL) return MX_ERR_SHAPE;
  constexpr auto kern = gemm_bf16_dma16s_kernel;
  MX_RETURN_IF_HIP(lds_limit_once<kern>(CF::LDS));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(CF::NT), CF::LDS, stream, (const uint16_t*)A,
                     (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

template <int NS, int WM, int WN, int BM_ = 256, int BN_ = 256>
static int launch_dma16(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                        hipStream_t stream) {
  using CF = D16Cfg<NS, WM, WN, BM_, BN_>;
  const long long tiles = (long long)((M + CF::BM - 1) / CF::BM) * ((N + CF::BN - 1) / CF::BN);
  if (tiles > 0x7fffffffLL) return MX_ERR_SHAPE;
  const int smem = NS * CF::STAGE;
  constexpr auto kern = gemm_bf16_dma16_kernel<NS, WM, WN, BM_, BN_>;
  MX_RETURN_IF_HIP(lds_limit_once<kern>(smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(CF::NT), smem, stream, (const uint16_t*)A,
                     (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

template <int BM, int BN, int WM, int WN, int KS = 1, int PF = 1>
static int launch(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                  hipStream_t stream, int batch = 1, long long sA = 0, long long sB = 0, long long sC = 0) {
  using CF = Cfg<BM, BN, WM, WN>;
  const long long tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7fffffffLL || batch > 65535) return MX_ERR_SHAPE;
  if (!staged_strides_ok<BM>(lda, ldb)) return MX_ERR_SHAPE;
  const size_t smem = (size_t)KS * 2 * CF::LDS_STAGE;
  static_assert(KS * 2 * CF::LDS_STAGE <= 160 * 1024, "double buffers fit in the LDS");
  constexpr auto kern = gemm_bf16_kernel<BM, BN, WM, WN, KS, PF>;
  MX_RETURN_IF_HIP(lds_limit_once<kern>((int)smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)batch), dim3(CF::NT * KS), smem, stream, (const uint16_t*)A,
                     (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

// ---------------------------------------------------------------------------
// Small-M batched kernel (M <= 32, e.g. one decode batch against one head's
// weight): weight-streaming, so it needs enough bytes in flight per CU and
// few rounds of workgroups rather than big tiles.  A workgroup is one wave
// computing a 32 x (32 NF) tile of C over the whole K; 64-deep chunks of A
// [32][64] and B [64][32 NF] go HBM -> LDS by direct loads into an
// NS-stage ring, NS-1 chunks ahead (6 stages for narrow tiles, 4 at NF = 4:
// 48-80 KB of LDS, two workgroups per CU).  A single wave needs no barrier: the ring stage
// it overwrites was consumed by its own MFMAs, which waited for those
// reads.  A rows (128 B) use the 16-row chunk swizzle of the large kernel;
// B rows (64 NF bytes) put chunk c of k-row k at c ^ (((k & 3) << 2) mod
// (4 NF)) so the 4 consecutive k-rows of a transposing read phase occupy
// distinct 64-byte quarters of the bank sweep (no swizzle needed at NF = 1,
// where those 4 rows are 256 contiguous bytes).
// ---------------------------------------------------------------------------
constexpr int SM_BK = 64;
constexpr int SM_A_B = 32 * SM_BK * 2;  // 4 KB

template <int NF>
__device__ __forceinline__ int sm_swz(int k) {
  return NF == 1 ? 0 : (((k & 3) << 2) & (4 * NF - 1));
}

// s_waitcnt for "at most min(MAXC, after) chunks of LPC loads in flight".
template <int LPC, int MAXC>
__device__ __forceinline__ void wait_chunks(int after) {
  if constexpr (MAXC >= 4) {
    if (after >= 4) { wait_vmcnt<4 * LPC>(); return; }
  }
  if constexpr (MAXC >= 3) {
    if (after == 3) { wait_vmcnt<3 * LPC>(); return; }
  }
  if constexpr (MAXC >= 2) {
    if (after == 2) { wait_vmcnt<2 * LPC>(); return; }
  }
  if (after >= 1) { wait_vmcnt<LPC>(); return; }
  wait_vmcnt<0>();
}

template <int NF>
__global__ __launch_bounds__(64) void gemm_bf16_smallm_kernel(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ B,
                                                              uint16_t* __restrict__ C, int M, int N, int K, int lda,
                                                              int ldb, int ldc, long long sA, long long sB,
                                                              long long sC) {
  constexpr int TN = 32 * NF;                 // columns per workgroup
  constexpr int RB = TN * 2;                  // B row bytes in LDS
  constexpr int B_B = SM_BK * RB;             // B chunk bytes
  constexpr int STAGE = SM_A_B + B_B;
  constexpr int BL = B_B / 1024;              // B direct loads per chunk
  constexpr int LPC = 4 + BL;                 // direct loads per chunk
  constexpr int BCH = RB / 16;                // 16-byte chunks per B row
  constexpr int BRPL = 1024 / RB;             // B rows per direct load
  constexpr int SM_NS = NF == 4 ? 4 : 6;      // ring stages
  __shared__ __align__(1024) unsigned char smem[SM_NS * STAGE];
  const int lane = threadIdx.x;
  const int g = lane >> 5;
  const int tiles_n = (N + TN - 1) / TN;
  const int n0 = (int)(blockIdx.x % tiles_n) * TN;
  const size_t item = blockIdx.x / tiles_n;
  A += item * sA;
  B += item * sB;
  C += item * sC;
  const int nk = K / SM_BK;
  const uint32_t lds0 = lds_addr(smem);

  // Direct-load lane offsets.  A load n (0..3): rows 8n + lane/8, chunk
  // (lane%8) ^ swz_a<64>(row); rows past M re-read row M-1.  B load n:
  // k-rows BRPL n + lane/BCH, chunk (lane%BCH) ^ sm_swz(k-row); columns
  // past N re-read the last valid 8.
  uint32_t a_off[4], b_off[BL];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int row = 8 * n + (lane >> 3);
    a_off[n] = (uint32_t)min(row, M - 1) * (uint32_t)lda * 2u + 16u * ((lane & 7) ^ swz_a<64>(row));
  }
#pragma unroll
  for (int n = 0; n < BL; ++n) {
    const int kr = BRPL * n + lane / BCH;
    const int col = min(n0 + 8 * ((lane % BCH) ^ sm_swz<NF>(kr)), N - 8);
    b_off[n] = (uint32_t)kr * (uint32_t)ldb * 2u + 2u * col;
  }
  auto issue = [&](int kt) {
    const uint32_t st = lds0 + (kt % SM_NS) * STAGE;
    const uint16_t* ab = A + (size_t)kt * SM_BK;
    const uint16_t* bb = B + (size_t)kt * SM_BK * ldb;
#pragma unroll
    for (int n = 0; n < 4; ++n) dma16(ab, a_off[n], st + n * 1024);
#pragma unroll
    for (int n = 0; n < BL; ++n) dma16(bb, b_off[n], st + SM_A_B + n * 1024);
  };

  // Fragments (C^T = B^T . A^T): A^T (B operand) row m = lane%32, chunk
  // 2 ks + g; B^T (A operand) of column tile nf by transposing reads, lane
  // (g, sg, 4j+a) at k-row 16 ks + 8 g + 4 r + j, columns 32 nf + 16 sg + 4 a.
  const int am = lane & 31;
  const int b_sg = (lane >> 4) & 1, b_j = (lane >> 2) & 3, b_a = lane & 3;
  const uint32_t a_base = lds0 + am * 128;
  const int ax = swz_a<64>(am);
  uint32_t b_base[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) {
    const int chunk = (32 * nf + 16 * b_sg + 4 * b_a) >> 3;  // k-row 8g + b_j: swizzle sm_swz(b_j)
    b_base[nf] = lds0 + SM_A_B + (8 * g + b_j) * RB + 16 * (chunk ^ sm_swz<NF>(b_j)) + 8 * (b_a & 1);
  }

  f32x16 acc[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) acc[nf] = f32x16{};
#pragma unroll
  for (int p = 0; p < SM_NS - 1; ++p)
    if (p < nk) issue(p);
  for (int kt = 0; kt < nk; ++kt) {
    // chunk kt landed once at most min(NS-2, nk-1-kt) later chunks are in flight
    wait_chunks<LPC, SM_NS - 2>(nk - 1 - kt);
    if (kt + SM_NS - 1 < nk) issue(kt + SM_NS - 1);
    const uint32_t so = (kt % SM_NS) * STAGE;
#pragma unroll
    for (int ks = 0; ks < SM_BK / 16; ++ks) {
      const u32x4 af = lds_ld128(a_base + so + 16 * ((2 * ks + g) ^ ax));
#pragma unroll
      for (int nf = 0; nf < NF; ++nf) {
        const uint32_t bp = b_base[nf] + so + 16 * ks * RB;
        const u32x2 lo = lds_read_tr16_at(bp);
        const u32x2 hi = lds_read_tr16_at(bp + 4 * RB);
        acc[nf] = mfma32<BF16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, af, acc[nf]);
      }
    }
  }

  // lane holds m = lane%32, n = n0 + 32 nf + 8 i + 4 g + {0..3}
  if (am < M) {
    uint16_t* crow = C + (size_t)am * ldc;
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gn = n0 + 32 * nf + 8 * i + 4 * g;
        const f32x16& a = acc[nf];
        if (gn < N) st64(crow + gn, u32x2{pack_bf16x2(a[4 * i], a[4 * i + 1]), pack_bf16x2(a[4 * i + 2], a[4 * i + 3])});
      }
  }
}

// Split-K variant for items with a few 64-deep K chunks (4..12, e.g. the
// 32 x 128 x 512 up-projection of the MLA absorbed step): one workgroup of
// KW waves per 32 x (32 NF) tile, wave w taking chunks w*nkw .. w*nkw +
// nkw - 1 and issuing all of them at once into its own LDS region, so a
// tile needs a single round trip to memory and reads A once per column
// tile; the partial sums meet in LDS (waves 1..KW-1 each write theirs into
// their own, consumed region, wave 0 adds and stores).
template <int NF, int KW>
__global__ __launch_bounds__(64 * KW) void gemm_bf16_smallm_sk_kernel(const uint16_t* __restrict__ A,
                                                                     const uint16_t* __restrict__ B,
                                                                     uint16_t* __restrict__ C, int M, int N, int K,
                                                                     int lda, int ldb, int ldc, long long sA,
                                                                     long long sB, long long sC) {
  constexpr int TN = 32 * NF, RB = TN * 2, B_B = SM_BK * RB, STAGE = SM_A_B + B_B;
  constexpr int BL = B_B / 1024, BCH = RB / 16, BRPL = 1024 / RB;
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;
  const int tiles_n = (N + TN - 1) / TN;
  const int n0 = (int)(blockIdx.x % tiles_n) * TN;
  const size_t item = blockIdx.x / tiles_n;
  A += item * sA;
  B += item * sB;
  C += item * sC;
  const int nkw = K / SM_BK / KW;  // chunks per wave (1..3)
  const int kc0 = wave * nkw;
  const uint32_t lds0 = lds_addr(smem) + wave * nkw * STAGE;

  // Direct-load lane offsets as in the kernel above.
  uint32_t a_off[4], b_off[BL];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int row = 8 * n + (lane >> 3);
    a_off[n] = (uint32_t)min(row, M - 1) * (uint32_t)lda * 2u + 16u * ((lane & 7) ^ swz_a<64>(row));
  }
#pragma unroll
  for (int n = 0; n < BL; ++n) {
    const int kr = BRPL * n + lane / BCH;
    const int col = min(n0 + 8 * ((lane % BCH) ^ sm_swz<NF>(kr)), N - 8);
    b_off[n] = (uint32_t)kr * (uint32_t)ldb * 2u + 2u * col;
  }
  for (int c = 0; c < nkw; ++c) {
    const uint32_t st = lds0 + c * STAGE;
    const uint16_t* ab = A + (size_t)(kc0 + c) * SM_BK;
    const uint16_t* bb = B + (size_t)(kc0 + c) * SM_BK * ldb;
#pragma unroll
    for (int n = 0; n < 4; ++n) dma16(ab, a_off[n], st + n * 1024);
#pragma unroll
    for (int n = 0; n < BL; ++n) dma16(bb, b_off[n], st + SM_A_B + n * 1024);
  }

  const int am = lane & 31;
  const int b_sg = (lane >> 4) & 1, b_j = (lane >> 2) & 3, b_a = lane & 3;
  const uint32_t a_base = lds0 + am * 128;
  const int ax = swz_a<64>(am);
  uint32_t b_base[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) {
    const int chunk = (32 * nf + 16 * b_sg + 4 * b_a) >> 3;
    b_base[nf] = lds0 + SM_A_B + (8 * g + b_j) * RB + 16 * (chunk ^ sm_swz<NF>(b_j)) + 8 * (b_a & 1);
  }
  f32x16 acc[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) acc[nf] = f32x16{};
  land_args(C);  // C is used only after the loop
  for (int c = 0; c < nkw; ++c) {
    // chunk c landed once at most nkw-1-c later chunks are in flight
    wait_chunks<4 + BL, 2>(nkw - 1 - c);
    const uint32_t so = c * STAGE;
#pragma unroll
    for (int ks = 0; ks < SM_BK / 16; ++ks) {
      const u32x4 af = lds_ld128(a_base + so + 16 * ((2 * ks + g) ^ ax));
#pragma unroll
      for (int nf = 0; nf < NF; ++nf) {
        const uint32_t bp = b_base[nf] + so + 16 * ks * RB;
        const u32x2 lo = lds_read_tr16_at(bp);
        const u32x2 hi = lds_read_tr16_at(bp + 4 * RB);
        acc[nf] = mfma32<BF16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, af, acc[nf]);
      }
    }
  }

  // Partial sums: waves 1..KW-1 into their own (consumed) LDS region, laid
  // out [nf][e][lane] so consecutive lanes hit consecutive banks.
  float* mine = reinterpret_cast<float*>(smem + wave * nkw * STAGE);
  if (wave > 0) {
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int e = 0; e < 16; ++e) mine[(nf * 16 + e) * 64 + lane] = acc[nf][e];
  }
  __syncthreads();
  if (wave > 0) return;  // no barrier follows
  for (int w = 1; w < KW; ++w) {
    const float* other = reinterpret_cast<const float*>(smem + w * nkw * STAGE);
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[nf][e] += other[(nf * 16 + e) * 64 + lane];
  }

  // lane holds m = lane%32, n = n0 + 32 nf + 8 i + 4 g + {0..3}
  if (am < M) {
    uint16_t* crow = C + (size_t)am * ldc;
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gn = n0 + 32 * nf + 8 * i + 4 * g;
        const f32x16& a = acc[nf];
        if (gn < N) st64(crow + gn, u32x2{pack_bf16x2(a[4 * i], a[4 * i + 1]), pack_bf16x2(a[4 * i + 2], a[4 * i + 3])});
      }
  }
}

static int launch_smallm(const void* A, const void* B, void* C, int batch, int M, int N, int K, int lda, int ldb,
                         int ldc, long long sA, long long sB, long long sC, hipStream_t stream) {
  auto groups = [&](int tn) { return (long long)batch * ((N + tn - 1) / tn); };
  // 4..12 chunks of K, split among 4 waves: one workgroup per 32 x 64 tile
  // when that still gives >= 256 workgroups (one per CU), else 32 x 32.
  const int nkc = K / SM_BK;
  if (nkc % 4 == 0 && nkc >= 4 && nkc <= 12) {
    const int nfs = groups(64) >= 256 ? 2 : 1;
    const long long gsk = groups(32 * nfs);
    if (gsk > 0x7fffffffLL) return MX_ERR_SHAPE;
    const int smem = nkc * (SM_A_B + SM_BK * 64 * nfs);
    if (nfs == 2) {
      constexpr auto kern = gemm_bf16_smallm_sk_kernel<2, 4>;
      MX_RETURN_IF_HIP(lds_limit_once<kern>(12 * (SM_A_B + SM_BK * 128)));
      hipLaunchKernelGGL(kern, dim3((unsigned)gsk), dim3(256), smem, stream, (const uint16_t*)A, (const uint16_t*)B,
                         (uint16_t*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
    } else {
      constexpr auto kern = gemm_bf16_smallm_sk_kernel<1, 4>;
      MX_RETURN_IF_HIP(lds_limit_once<kern>(12 * (SM_A_B + SM_BK * 64)));
      hipLaunchKernelGGL(kern, dim3((unsigned)gsk), dim3(256), smem, stream, (const uint16_t*)A, (const uint16_t*)B,
                         (uint16_t*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
    }
    MX_RETURN_IF_HIP(hipGetLastError());
    return MX_OK;
  }
  // Widest column tile that still leaves >= 512 workgroups (two per CU).
  const int nf = groups(128) >= 512 ? 4 : (groups(64) >= 512 ? 2 : 1);
  const long long grid = groups(32 * nf);
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  if (nf == 4)
    hipLaunchKernelGGL(gemm_bf16_smallm_kernel<4>, dim3((unsigned)grid), dim3(64), 0, stream, (const uint16_t*)A,
                       (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
  else if (nf == 2)
    hipLaunchKernelGGL(gemm_bf16_smallm_kernel<2>, dim3((unsigned)grid), dim3(64), 0, stream, (const uint16_t*)A,
                       (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
  else
    hipLaunchKernelGGL(gemm_bf16_smallm_kernel<1>, dim3((unsigned)grid), dim3(64), 0, stream, (const uint16_t*)A,
                       (const uint16_t*)B, (uint16_t*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}


// ---------------------------------------------------------------------------
// gemm_bf16_stream_kernel: products with few tiles (decode batches, small
// M or N with a long K) stream the weights B.  Tiles of 64 or more rows
// would leave most CUs idle.
//  * A workgroup owns 32 columns x 32 MF rows of C, NW waves; wave w takes
//    the 64-deep K blocks kb = w, w + NW, ..., so every workgroup streams its
//    32 columns of B once.  The row chunks of a column block and the
//    neighbouring column blocks run on one XCD, where they share B's
//    128-byte lines in L2.
//  * Each wave has a private ring of NSL slots, one K block per slot (A: 32 MF
//    rows x 128 B, chunk c at c ^ ((m >> 1) & 7); B: 64 k-rows x 64 B), by
//    direct loads; slots are private, so the block loop has no barrier.
//  * C^T = B^T . A^T on 32x32x16 MFMAs: B^T fragments by transposing reads
//    from the 64-byte B rows (a 32-lane phase covers 4 rows x 64 B, conflict
//    free unswizzled), A^T fragments by ds_read_b128.
//  * The waves' accumulators meet in LDS at the end; wave i sums and stores
//    the four result registers holding n = 8i + 4(l/32) + {0..3}.
// ---------------------------------------------------------------------------
template <int MF, int NW, int NSL>
struct StreamCfg {
  static constexpr int A_B = 32 * MF * 128;  // 64 k of 32 MF rows
  static constexpr int B_B = 64 * 64;         // 64 k-rows of 32 columns
  static constexpr int SLOT = A_B + B_B;
  static constexpr int A_L = A_B / 1024, B_L = B_B / 1024;
  static constexpr int VM = A_L + B_L;
  static constexpr int LDS = NW * NSL * SLOT;
  static_assert(NW == 4, "one reducing wave per result register quad");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert((NSL - 1) * VM < 64, "vmcnt range");
  static_assert(NW * MF * 64 * 16 * 4 <= LDS, "reduction area");
};
__device__ __forceinline__ int swz_s(int m) { return (m >> 1) & 7; }
// f(integral_constant<int, I>) for I = 0 .. N-1, in order.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void unroll_n(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    unroll_n<N, I + 1>(f);
  }
}

template <int MF, int NW, int NSL>
__global__ __launch_bounds__(64 * NW, 1) void gemm_bf16_stream_kernel(const uint16_t* __restrict__ A,
                                                                    const uint16_t* __restrict__ B,
                                                                    uint16_t* __restrict__ C, int M, int N, int K,
                                                                    int lda, int ldb, int ldc) {
  using CF = StreamCfg<MF, NW, NSL>;
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Workgroup -> (32-column block, chunk of 32 MF rows), the row chunks of a
  // column block adjacent, so one XCD holds whole column blocks and their
  // neighbours (which share B's lines in L2).
  const int nmc = (M + 32 * MF - 1) / (32 * MF);
  const int wid = xcd_remap(blockIdx.x, (int)gridDim.x);
  const int n0 = (wid / nmc) * 32, m0 = (wid % nmc) * 32 * MF;
  A += (size_t)m0 * lda;
  C += (size_t)m0 * ldc;
  M -= m0;  // rows of this chunk (more than 32 MF only past the last row read)
  const int kblocks = K / 64;
  const int cnt = kblocks > wave ? (kblocks - wave + NW - 1) / NW : 0;
  const uint32_t ring = lds_addr(smem) + wave * NSL * CF::SLOT;

  // A load n: rows 8n + l/8, LDS chunk l%8 taking global chunk (l%8) ^
  // swz(row) (rows past M re-read row M-1); B load n: k-rows 16n + l/4,
  // chunk l%4 (columns past N re-read the last 8 valid ones; never stored).
  uint32_t a_off[CF::A_L], b_off[CF::B_L];
#pragma unroll
  for (int n = 0; n < CF::A_L; ++n) {
    const int row = 8 * n + (lane >> 3);
    a_off[n] = (uint32_t)min(row, M - 1) * (uint32_t)lda * 2u + 16u * ((lane & 7) ^ swz_s(row));
  }
#pragma unroll
  for (int n = 0; n < CF::B_L; ++n) {
    const int col = min(n0 + 8 * (lane & 3), N - 8) - n0;
    b_off[n] = (uint32_t)(16 * n + (lane >> 2)) * (uint32_t)ldb * 2u + 2u * col;
  }
  auto issue = [&](int i, auto slot_tag) {
    constexpr int I = decltype(slot_tag)::value;
    const int kb = cnt > 0 ? wave + NW * min(i, cnt - 1) : 0;
    const uint32_t st = ring + I * CF::SLOT;
#pragma unroll
    for (int n = 0; n < CF::A_L; ++n) dma16(A + (size_t)kb * 64, a_off[n], st + n * 1024);
#pragma unroll
    for (int n = 0; n < CF::B_L; ++n) dma16(B + (size_t)kb * 64 * ldb + n0, b_off[n], st + CF::A_B + n * 1024);
  };

  // fragment lane addresses within a slot.  A^T (B operand): row am, chunk
  // 2 ks + g.  B^T (A operand): lane 16G + 4j + a reads k-row 8 (G>>1) +
  // 4 r + j (+16 ks), columns 16 (G&1) + 4a .. +3.
  const int am = lane & 31, g = lane >> 5;
  uint32_t a_col[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) a_col[ks] = am * 128 + 16 * ((2 * ks + g) ^ swz_s(am));
  const int G = lane >> 4, bj = (lane >> 2) & 3, ba = lane & 3;
  const uint32_t b_col = CF::A_B + (8 * (G >> 1) + bj) * 64 + 32 * (G & 1) + 8 * ba;

  f32x16 acc[MF];
#pragma unroll
  for (int f = 0; f < MF; ++f) acc[f] = f32x16{};

  auto compute = [&](auto slot_tag) {
    constexpr int I = decltype(slot_tag)::value;
    const uint32_t st = ring + I * CF::SLOT;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x2 lo = lds_read_tr16_at(st + b_col + 16 * ks * 64);
      const u32x2 hi = lds_read_tr16_at(st + b_col + 16 * ks * 64 + 4 * 64);
      const u32x4 bt{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int f = 0; f < MF; ++f) acc[f] = mfma32<BF16>(bt, lds_ld128(st + 32 * f * 128 + a_col[ks]), acc[f]);
    }
  };

  land_args(C);
  unroll_n<NSL - 1>([&](auto i_tag) { issue(decltype(i_tag)::value, i_tag); });
  // block i: issue block i + NSL - 1 into the slot block i - 1 used (its
  // reads completed), then wait for block i
  auto step = [&](int i, auto slot_tag) {
    constexpr int I = decltype(slot_tag)::value;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    issue(i + NSL - 1, std::integral_constant<int, (I + NSL - 1) % NSL>{});
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NSL - 1) * CF::VM) : "memory");
    compute(slot_tag);
  };
  int i = 0;
  for (; i + NSL <= cnt; i += NSL) unroll_n<NSL>([&](auto s_tag) { step(i + decltype(s_tag)::value, s_tag); });
  unroll_n<NSL - 1>([&](auto s_tag) {
    if (i + decltype(s_tag)::value < cnt) step(i + decltype(s_tag)::value, s_tag);
  });
  wait_vmcnt<0>();  // no DMA may land in the ring once it is reused below

  // ---- accumulators meet in LDS: [wave][f][e][lane] floats ----
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int f = 0; f < MF; ++f)
#pragma unroll
    for (int e = 0; e < 16; ++e) red[((wave * MF + f) * 16 + e) * 64 + lane] = acc[f][e];
  __syncthreads();
  const int gn = n0 + 8 * wave + 4 * g;
#pragma unroll
  for (int f = 0; f < MF; ++f) {
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += red[((w * MF + f) * 16 + 4 * wave + j) * 64 + lane];
    const int gm = 32 * f + am;
    if (gm < M && gn < N)
      st64(C + (size_t)gm * ldc + gn, u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])});
  }
}

template <int MF, int NSL>
static int launch_stream(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb, int ldc,
                         hipStream_t stream) {
  using CF = StreamCfg<MF, 4, NSL>;
  constexpr auto kern = gemm_bf16_stream_kernel<MF, 4, NSL>;
  MX_RETURN_IF_HIP(lds_limit_once<kern>(CF::LDS));
  const long long grid = (long long)((N + 31) / 32) * ((M + 32 * MF - 1) / (32 * MF));
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), CF::LDS, stream, (const uint16_t*)A,
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
  // Stream the weights with whole 64-deep K blocks (32-bit lane offsets: 64
  // rows of A and 64 k-rows of B span < 4 GiB) for decode-sized M against
  // at least 256 columns, and for any product with at most 64 tiles of
  // 64x64 and K >= 512, which the tiled kernels cannot spread over the CUs
  // (graph-replayed: 256x512x4096 17.6 -> 9.4 us, 96x512x8192 44.9 -> 14.4
  // us; 1024^3, 256 such tiles, stays tiled: 8.3 against 10.6 us).
  const long long tiles64s = (long long)((M + 63) / 64) * ((N + 63) / 64);
  if (((M <= 64 && N >= 256) || (tiles64s <= 64 && K >= 512)) && K % 64 == 0 &&
      (long long)lda * 2 * 64 <= 0xffffffffLL && (long long)ldb * 2 * 64 <= 0xffffffffLL)
    return M <= 32 ? mx::gemm::launch_stream<1, 4>(A, B, C, M, N, K, lda, ldb, ldc, s)
                   : mx::gemm::launch_stream<2, 3>(A, B, C, M, N, K, lda, ldb, ldc, s);
  const long long tiles256 = (long long)((M + 255) / 256) * ((N + 255) / 256);
  const long long tiles128 = (long long)((M + 127) / 128) * ((N + 127) / 128);
  // Rounds of 256 workgroups: a round of 256x256 tiles of the direct-load
  // kernel takes ~2.6 times a round of its 128x128 tiles at the same K
  // (measured 2.2-3.0 at 2048-4096), so 256x256 also wins below one tile
  // per CU when 128x128 tiles would need more than 2.6 times the rounds
  // (3072^3: 69 vs 78 us; 2560^3 stays on 128x128: 48 vs 59 us).
  const long long r256 = (tiles256 + 255) / 256, r128 = (tiles128 + 255) / 256;
  const bool big = tiles256 >= 256 || 13 * r256 < 5 * r128;
  // Whole K tiles: the direct-load kernel (its lane offsets are 32-bit: 256
  // rows of A must span < 4 GiB).
  if (big && K % 64 == 0 && (long long)lda * 2 * 256 <= 0xffffffffLL && (long long)ldb * 2 * 32 <= 0xffffffffLL)
    return mx::gemm::launch_dma16s(A, B, C, M, N, K, lda, ldb, ldc, s);
  if (big && K % mx::gemm::DMA_BK == 0 && (long long)lda * 2 * 256 <= 0xffffffffLL)
    return mx::gemm::launch_dma16<mx::gemm::DMA_NS, mx::gemm::DMA_WM, mx::gemm::DMA_WN>(A, B, C, M, N, K, lda, ldb,
                                                                                          ldc, s);
  // Otherwise: register-staged kernels, big tiles when they still cover the
  // 256 CUs twice, else smaller tiles for parallelism.
  if (tiles256 >= 512) return mx::gemm::launch<256, 256, 2, 4>(A, B, C, M, N, K, lda, ldb, ldc, s);
  // At least one 128x128 tile per CU and whole K tiles: the direct-load
  // kernel on 128x128 tiles, whose 16 KB stages allow a deeper ring.
  if (tiles128 >= 256 && K % mx::gemm::DMA_BK == 0 && (long long)lda * 2 * 128 <= 0xffffffffLL)
    return mx::gemm::launch_dma16<mx::gemm::D128_NS, 2, mx::gemm::D128_WN, 128, 128>(A, B, C, M, N, K, lda, ldb,
                                                                                      ldc, s);
  if (tiles128 >= 256) return mx::gemm::launch<128, 128, 2, 2>(A, B, C, M, N, K, lda, ldb, ldc, s);
  // About one 64x64 tile per CU or fewer and a long K (e.g. 1024^3): split
  // K between two wave groups of each workgroup.
  const long long tiles64 = (long long)((M + 63) / 64) * ((N + 63) / 64);
  // ... with whole 64x64 tiles and 128-deep K chunks: the direct-load ring
  // (32-bit lane offsets: 64 rows of A and 64 k-rows of B span < 4 GiB).
  if (tiles64 <= 256 && K >= 512 && M % 64 == 0 && N % 64 == 0 && K % 128 == 0 &&
      (long long)lda * 2 * 64 <= 0xffffffffLL && (long long)ldb * 2 * 64 <= 0xffffffffLL)
    return mx::gemm::launch_sdma(A, B, C, M, N, K, lda, ldb, ldc, s);
  if (tiles64 <= 256 && K >= 512) return mx::gemm::launch<64, 64, 2, 2, 2, 2>(A, B, C, M, N, K, lda, ldb, ldc, s);
  return mx::gemm::launch<64, 64, 2, 2, 1, 2>(A, B, C, M, N, K, lda, ldb, ldc, s);
}

namespace mx {
namespace gemm {

// Which kernel mx_gemm_bf16_batched runs for these sizes.
enum class BatchedPath { SmallM, T128, T64 };

static BatchedPath batched_path(int batch, int M, int N, int K, int lda, int ldb) {
  // Decode-sized items (M <= 32, whole 64-deep K chunks): the
  // weight-streaming small-M kernel.  Its lane offsets are 32-bit.
  if (M <= 32 && K % 64 == 0 && (long long)lda * 2 * 32 <= 0xffffffffLL && (long long)ldb * 2 * 64 <= 0xffffffffLL)
    return BatchedPath::SmallM;
  // Otherwise the register-staged kernel with tiles sized to the item.
  const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128) * batch;
  if (M >= 128 && t128 >= 256) return BatchedPath::T128;
  return BatchedPath::T64;
}

// Every check mx_gemm_bf16_batched makes before it launches, the grid
// limits of the kernel it would pick included, so a caller that chains
// several products can validate them all before enqueuing any.
int batched_check(const void* A, const void* B, void* C, int batch, int M, int N, int K, int lda, int ldb, int ldc,
                  long long strideA, long long strideB, long long strideC) {
  if (!A || !B || !C) return MX_ERR_NULL;
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0) return MX_ERR_SHAPE;
  if (batch > 65535 || strideA < 0 || strideB < 0 || strideC < 0) return MX_ERR_SHAPE;
  if (lda < K || ldb < N || ldc < N) return MX_ERR_SHAPE;
  if ((K % 8) || (N % 8) || (lda % 8) || (ldb % 8) || (ldc % 8)) return MX_ERR_ALIGN;
  if ((strideA % 8) || (strideB % 8) || (strideC % 8)) return MX_ERR_ALIGN;
  if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return MX_ERR_ALIGN;
  long long grid = 0;
  switch (batched_path(batch, M, N, K, lda, ldb)) {
    case BatchedPath::SmallM: grid = (long long)batch * ((N + 31) / 32); break;  // widest grid of the three widths
    case BatchedPath::T128:
      grid = (long long)((M + 127) / 128) * ((N + 127) / 128);
      if (!staged_strides_ok<128>(lda, ldb)) return MX_ERR_SHAPE;
      break;
    case BatchedPath::T64:
      grid = (long long)((M + 63) / 64) * ((N + 63) / 64);
      if (!staged_strides_ok<64>(lda, ldb)) return MX_ERR_SHAPE;
      break;
  }
  return grid > 0x7fffffffLL ? MX_ERR_SHAPE : MX_OK;
}

}  // namespace gemm
}  // namespace mx

extern "C" int mx_gemm_bf16_batched(const void* A, const void* B, void* C, int batch, int M, int N, int K, int lda,
                                    int ldb, int ldc, long long strideA, long long strideB, long long strideC,
                                    void* stream) {
  using namespace mx::gemm;
  if (const int e = batched_check(A, B, C, batch, M, N, K, lda, ldb, ldc, strideA, strideB, strideC)) return e;
  hipStream_t s = (hipStream_t)stream;
  switch (batched_path(batch, M, N, K, lda, ldb)) {
    case BatchedPath::SmallM:
      return launch_smallm(A, B, C, batch, M, N, K, lda, ldb, ldc, strideA, strideB, strideC, s);
    case BatchedPath::T128:
      return launch<128, 128, 2, 2>(A, B, C, M, N, K, lda, ldb, ldc, s, batch, strideA, strideB, strideC);
    default:
      return launch<64, 64, 2, 2, 1, 2>(A, B, C, M, N, K, lda, ldb, ldc, s, batch, strideA, strideB, strideC);
  }
}
