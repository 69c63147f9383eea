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
//    power-of-two E8M0 hardware scales cannot carry them).  Each fragment's
//    two MFMAs issue back to back and the previous fragment's promotion
//    follows them, so its FMAs run while those two MFMAs execute.
//  * 256x256 tiles, 8 waves (2 in m x 4 in n, two per SIMD), each wave
//    128(m) x 64(n): the fp32 accumulators stay in architectural VGPRs,
//    where the promotion FMAs can reach them.  Grids under 256 such tiles
//    use 128x128 tiles.
//  * A and B go HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging),
//    filling the 160 KB of LDS with two rings: A in whole scale blocks (BM
//    rows of 128 bytes, so every load request is a full 128-byte line; rows
//    of 64 bytes made each line two half-line requests, which kept the L1
//    address path stalled) in 3 slots, issued two blocks ahead; B in
//    64-deep stages (64 k-rows of BN bytes, whole lines already) in 4
//    slots, one block ahead.  One barrier per scale block.  Every block
//    issues the same loads (past the end, the last block again into slots
//    nobody reads), so the wait counts never vary.
//  * The block scales are read with vector loads issued as inline asm and
//    waited for by the same vmcnt wait that lands the stages, as operands
//    of that wait: the compiler tracks neither, so it never inserts a
//    vmcnt(0) of its own that would drain the ring.  When K is a multiple
//    of 512 the activation scales come four blocks per 8-byte load (the
//    two half-waves take blocks 4g, 4g+1 and 4g+2, 4g+3 of the rows they
//    share), once per four blocks: one scale per lane per block made each
//    block's scale loads touch more cache lines than its A and B tiles.
//  * A^T fragments are plain ds_read_b128; B^T fragments come from k-major
//    B rows through gfx950's transposing read ds_read_b64_tr_b8: in each
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

constexpr int SBK = 128;   // bytes of K per scale block (= per A slot)
constexpr int BKS = 64;    // bytes of K per B stage (one 32x32x64 k-step)
constexpr int NSA = 3;     // A ring slots (whole scale blocks)
constexpr int NSB = 4;     // B ring slots (half scale blocks)
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

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// A 4-byte vector load the compiler does not track (see the file comment):
// the result may only be read after a wait_scales() that names it.
__device__ __forceinline__ float ld_scale(const float* sbase, uint32_t voff) {
  float x;
  asm volatile("global_load_dword %0, %1, %2" : "=v"(x) : "v"(voff), "s"(sbase) : "memory");
  return x;
}
// Untracked 8-byte scale loads (two consecutive scales each, otherwise as
// ld_scale) issued only when `go` is nonzero, with the branch inside the
// statement: the registers are read-write operands, so they keep their
// values when the loads are skipped and the compiler sees no control flow
// (a branch around the loads split the registers' live ranges, and the
// allocator then copied an in-flight one).
__device__ __forceinline__ void ld_scales_if(u32x2 (&x)[4], const float* sbase, const uint32_t (&voff)[4],
                                             uint32_t go) {
  asm volatile(
      "s_cmp_eq_u32 %[go], 0\n\t"
      "s_cbranch_scc1 1f\n\t"
      "global_load_dwordx2 %0, %4, %[b]\n\t"
      "global_load_dwordx2 %1, %5, %[b]\n\t"
      "global_load_dwordx2 %2, %6, %[b]\n\t"
      "global_load_dwordx2 %3, %7, %[b]\n"
      "1:"
      : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3])
      : "v"(voff[0]), "v"(voff[1]), "v"(voff[2]), "v"(voff[3]), [b] "s"(sbase), [go] "s"(go)
      : "memory", "scc");
}
__device__ __forceinline__ void ld_scales_if(u32x2 (&x)[2], const float* sbase, const uint32_t (&voff)[2],
                                             uint32_t go) {
  asm volatile(
      "s_cmp_eq_u32 %[go], 0\n\t"
      "s_cbranch_scc1 1f\n\t"
      "global_load_dwordx2 %0, %2, %[b]\n\t"
      "global_load_dwordx2 %1, %3, %[b]\n"
      "1:"
      : "+v"(x[0]), "+v"(x[1])
      : "v"(voff[0]), "v"(voff[1]), [b] "s"(sbase), [go] "s"(go)
      : "memory", "scc");
}
// s_waitcnt vmcnt(N) that also lands the untracked scale loads: the scale
// registers are operands, so no read of them is scheduled before it.
template <int N, typename S, int FM>
__device__ __forceinline__ void wait_scales(S (&sa)[FM], float& sb) {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  static_assert(FM == 2 || FM == 4, "scale registers");
  if constexpr (FM == 4)
    asm volatile("s_waitcnt vmcnt(%5)" : "+v"(sa[0]), "+v"(sa[1]), "+v"(sa[2]), "+v"(sa[3]), "+v"(sb) : "i"(N)
                 : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%3)" : "+v"(sa[0]), "+v"(sa[1]), "+v"(sb) : "i"(N) : "memory");
}
#pragma clang diagnostic pop

template <int BM, int BN>
struct Cfg {
  static constexpr int WM = 2, WN = 4;
  static constexpr int TM = BM / WM, TN = BN / WN;   // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;   // 32x32 fragments
  static constexpr int A_S = BM * SBK;               // A slot: BM rows of 128 B (one scale block)
  static constexpr int B_S = BKS * BN;               // B slot: 64 k-rows of BN B
  static constexpr int B_OFF = NSA * A_S;            // the B ring follows the A ring
  static constexpr int LDS = NSA * A_S + NSB * B_S;
  static constexpr int A_LPW = A_S / 1024 / NWAVES;  // 1 KB direct loads per wave per A block
  static constexpr int B_LPW = B_S / 1024 / NWAVES;  // ... per B stage
  static constexpr int A_RPL = 1024 / SBK;           // A rows per 1 KB load
  static constexpr int B_CH = BN / 16;               // 16-byte chunks per B row
  static constexpr int B_RPL = 1024 / BN;            // B rows per 1 KB load
  static_assert(FM >= 1 && FN >= 1 && A_LPW >= 1 && B_LPW >= 1, "tile split");
  static_assert(TN <= 128 && 128 % TN == 0, "a wave's columns share one weight-scale block");
  static_assert(BN == 128 || BN == 256, "B row swizzle");
  static_assert(LDS <= 160 * 1024, "LDS ring");
};

// Chunk position swizzles.  A rows (128 B, 8 chunks): a 16-lane b128 phase
// reads one chunk of 16 consecutive rows, two rows per 256 B, so the
// position takes (m/2)%8.  B rows: a 32-lane transposing phase reads 8
// consecutive k-rows x 2 adjacent chunks.
__device__ __forceinline__ int swz_a(int m) { return (m >> 1) & 7; }
template <int BN>
__device__ __forceinline__ int swz_b(int k) {
  return BN == 256 ? ((k & 7) << 1) : (((k >> 1) & 3) << 1);
}

// GS (K a multiple of 512): the activation scales are loaded four blocks
// at a time (see load_sa), else one block at a time.
template <int BM, int BN, bool GS>
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
  const int kblocks = K / SBK;
  const int nst = 2 * kblocks;  // 64-byte stages
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
    const int row = CF::A_RPL * (wave * CF::A_LPW + n) + (lane >> 3);
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
  const uint8_t* a_tile = A + (size_t)m0 * K;
  const uint8_t* b_tile = B + n0;
  // Part n of A block j (128 bytes of K: whole 128-byte lines of every row)
  // into A slot j % NSA, and of B stage s (64 bytes of K) into B slot
  // s % NSB.  Blocks and stages past the end re-load the last one (into a
  // slot no later block reads).
  auto issue_a = [&](int j, int n) {
    const int src = min(j, kblocks - 1);
    dma16(a_tile + (size_t)src * SBK, a_off[n], lds0 + (j % NSA) * CF::A_S + (wave * CF::A_LPW + n) * 1024);
  };
  auto issue_b = [&](int s, int n) {
    const int src = min(s, nst - 1);
    dma16(b_tile + (size_t)src * BKS * N, b_off[n],
          lds0 + CF::B_OFF + (s % NSB) * CF::B_S + (wave * CF::B_LPW + n) * 1024);
  };

  // ---- fragment lane addresses in the first slot of each ring ----
  // A^T (B operand): row m = wm*TM + 32 mf + l%32, chunks 4 kh + 2 (l/32)
  // + {0,1} for the block's k half kh.
  const int am = wm * CF::TM + (lane & 31);
  const int a_x = swz_a(am);  // the same for every mf (32 rows apart)
  uint32_t a_col[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h) a_col[kh][h] = lds0 + am * SBK + 16 * ((4 * kh + 2 * (lane >> 5) + h) ^ a_x);
  // B^T (A operand) via tr_b8: in 16-lane group q, lane 2j+h reads k-row
  // 32 (q>>1) + 8 r + j, columns wn*TN + 32 nf + 16 (q&1) + 8 h.
  const int q = lane >> 4, jj = (lane & 15) >> 1, hh = lane & 1;
  const int b_k0 = 32 * (q >> 1) + jj;                       // plus 8 r
  const int b_c0 = wn * CF::TN + 16 * (q & 1) + 8 * hh;      // plus 32 nf
  const int b_x = swz_b<BN>(b_k0);  // rows 8 apart share it
  uint32_t b_col[FN];
#pragma unroll
  for (int nf = 0; nf < FN; ++nf) {
    const int col = b_c0 + 32 * nf;
    b_col[nf] = lds0 + CF::B_OFF + b_k0 * BN + 16 * ((col >> 4) ^ b_x) + (col & 15);
  }

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};

  // Block scales: the sA row of this lane per m fragment, the sB of this
  // wave's 128-column block (wave-uniform, read by every lane).  A wave's
  // 32 rows per m fragment lie 4 K/128 bytes apart, so a load of one scale
  // per lane touches 32 cache lines for 128 useful bytes; per block that
  // was more L1 lookups than the block's A and B tiles.  With GS the two
  // half-waves (lanes l and l + 32 share a row) load blocks 4g, 4g+1 and
  // 4g+2, 4g+3 of their row with one 8-byte load, once per four blocks,
  // and a v_permlane32_swap hands each lane the scale of the current block.
  uint32_t sa_off[FM];
#pragma unroll
  for (int mf = 0; mf < FM; ++mf)
    sa_off[mf] = (uint32_t)min(m0 + am + 32 * mf, M - 1) * (uint32_t)kblocks * 4u + (GS ? 8u * (lane >> 5) : 0u);
  const uint32_t sb_off = (uint32_t)min((n0 + wn * CF::TN) / 128, nblocks_n - 1) * 4u;
  std::conditional_t<GS, u32x2, float> sa_n[FM];
  float sb_n;
  auto load_sb = [&](int j) { sb_n = ld_scale(sB + (size_t)min(j, kblocks - 1) * nblocks_n, sb_off); };
  auto load_sa = [&](int j) {  // GS: at j = 4g - 1, group g (blocks 4g .. 4g+3)
    if constexpr (GS) {
      ld_scales_if(sa_n, sA + min(j + 1, kblocks - 4), sa_off, (uint32_t)(((j & 3) + 1) >> 2));  // 1 at j % 4 == 3
    } else {
      const int jb = min(j, kblocks - 1);
#pragma unroll
      for (int mf = 0; mf < FM; ++mf) sa_n[mf] = ld_scale(sA + jb, sa_off[mf]);
    }
  };
  // The activation scale of block 4g + t (GS; else of the loaded block)
  // for this lane's row in m fragment mf.
  auto sa_of = [&](int t, int mf) {
    if constexpr (GS) {
      const uint32_t v = (t & 1) ? sa_n[mf][1] : sa_n[mf][0];
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return __uint_as_float(t < 2 ? r[0] : r[1]);  // r[0]: lanes 0-31's value, r[1]: lanes 32-63's
    } else {
      return sa_n[mf];
    }
  };

  auto read_b = [&](uint32_t so, int nf) {
    u32x2 v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = lds_read_tr8_at(b_col[nf] + so + 8 * r * BN);
    return i32x8{(int)v[0][0], (int)v[0][1], (int)v[1][0], (int)v[1][1],
                 (int)v[2][0], (int)v[2][1], (int)v[3][0], (int)v[3][1]};
  };
  auto read_a = [&](uint32_t so, int kh, int mf) {
    const uint32_t r = so + 32 * mf * SBK;
    const u32x4 lo = lds_ld128(a_col[kh][0] + r);
    const u32x4 hi = lds_ld128(a_col[kh][1] + r);
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };

  land_args(C);  // C is used only after the loop

  // Prologue, in the order the block waits need: the scales of block 0,
  // A block 0, B stages 0 and 1, then A block 1 (which may still be in
  // flight when block 0 starts).
  load_sb(0);
  load_sa(GS ? -1 : 0);  // GS: group 0 (blocks 0 .. 3)
#pragma unroll
  for (int n = 0; n < CF::A_LPW; ++n) issue_a(0, n);
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int n = 0; n < CF::B_LPW; ++n) issue_b(s, n);
#pragma unroll
  for (int n = 0; n < CF::A_LPW; ++n) issue_a(1, n);

  // Scale block j: A block j and B stages 2j, 2j+1.  The two MFMAs of each
  // fragment build a fresh fp32 partial over the block's 128 k, promoted
  // with one FMA per element after the next fragment's two MFMAs:
  // acc += (sA sB) * partial.  The block's loads (B stages 2j+2, 2j+3, then
  // A block j+2) are issued spread over the row blocks.
  for (int j = 0; j < kblocks; ++j) {
    // A block j, B stages 2j, 2j+1 and the scales of block j landed (only A
    // block j+1 may be in flight); after the barrier every wave has
    // finished block j-1, so its A slot and B slots take the new loads.
    wait_scales<CF::A_LPW>(sa_n, sb_n);
    lds_barrier();
    float s_m[FM];
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) s_m[mf] = sa_of(j & 3, mf) * sb_n;
    // the next block's scales, issued before the block's tile loads so the
    // next block's wait lands them (GS: the next group's, once per group)
    load_sb(j + 1);
    if constexpr (GS) load_sa(j);
    else load_sa(j + 1);
    const uint32_t ao = (j % NSA) * CF::A_S;
    const uint32_t so0 = ((2 * j) % NSB) * CF::B_S, so1 = ((2 * j + 1) % NSB) * CF::B_S;

    // Issue order (pinned by sched barriers): each fragment's two MFMAs
    // back to back, then the promotion of the fragment before it, so its
    // FMAs wait only for an MFMA that finished while the next fragment's
    // two were queued (an FMA group between the two MFMAs of a fragment
    // leaves the MFMA pipe idle while it issues).  At most ~10 LDS reads in
    // flight (lgkmcnt counts 15); a partial is rewritten only after its FMAs
    // issued; a row block's A fragments are refilled once their last MFMA
    // issued.
    i32x8 bf0[FN], bf1[FN], a0, a1;
    f32x16 p[2];  // partials of consecutive fragments (mf, nf) in turn
    bf0[0] = read_b(so0, 0);
    a0 = read_a(ao, 0, 0);
    bf1[0] = read_b(so1, 0);
    a1 = read_a(ao, 1, 0);
    __builtin_amdgcn_sched_barrier(0);
    auto promote = [&](int nf, int mf) { acc[nf][mf] += s_m[mf] * p[(mf * FN + nf) & 1]; };
    constexpr int NLD = 2 * CF::B_LPW + CF::A_LPW;  // loads per block and wave
    auto dma_share = [&](int mf) {
#pragma unroll
      for (int n = (NLD * mf) / FM; n < (NLD * (mf + 1)) / FM; ++n) {
        if (n < 2 * CF::B_LPW)
          issue_b(2 * j + 2 + n / CF::B_LPW, n % CF::B_LPW);
        else
          issue_a(j + 2, n - 2 * CF::B_LPW);
      }
    };
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) {
#pragma unroll
      for (int nf = 0; nf < FN; ++nf) {
        f32x16& pp = p[(mf * FN + nf) & 1];
        pp = mfma32_fp8(bf0[nf], a0, f32x16{});
        __builtin_amdgcn_sched_barrier(0);
        if (mf == 0 && nf + 1 < FN) {
          bf0[nf + 1] = read_b(so0, nf + 1);
          bf1[nf + 1] = read_b(so1, nf + 1);
        }
        if (nf == FN - 1) {
          if (mf + 1 < FM) a0 = read_a(ao, 0, mf + 1);
          dma_share(mf);
        }
        __builtin_amdgcn_sched_barrier(0);
        pp = mfma32_fp8(bf1[nf], a1, pp);
        __builtin_amdgcn_sched_barrier(0);
        if (nf == FN - 1 && mf + 1 < FM) a1 = read_a(ao, 1, mf + 1);
        if (nf > 0)
          promote(nf - 1, mf);
        else if (mf > 0)
          promote(FN - 1, mf - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    promote(FN - 1, FM - 1);  // the block's last fragment
  }
  wait_scales<0>(sa_n, sb_n);  // no DMA may land in LDS after the workgroup ends

  // ---- store C through LDS.  Lane results are runs of four n of one row
  // (8 bytes), so direct stores would write each row of the tile in 16-byte
  // pieces from eight instructions, which the memory system writes back as
  // partial lines.  Instead the tile goes to LDS as bf16 rows (padded by
  // 16 bytes so the 32 rows of a fragment store land on distinct bank
  // slots), and the workgroup then writes whole rows, each lane 16
  // contiguous bytes.  The ring is free: every DMA has landed (vmcnt(0)
  // above) and the barrier below waits for every wave's last fragment
  // reads. ----
  constexpr int CROW = BN * 2 + 16;  // LDS bytes per staged C row
  static_assert(BM * CROW <= CF::LDS, "C tile fits the ring");
  __syncthreads();
  {
    unsigned char* ct = smem;
#pragma unroll
    for (int mf = 0; mf < FM; ++mf) {
      const int r = am + 32 * mf;  // tile row
#pragma unroll
      for (int nf = 0; nf < FN; ++nf)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = wn * CF::TN + 32 * nf + 8 * i + 4 * (lane >> 5);  // tile column
          const f32x16& a = acc[nf][mf];
          *reinterpret_cast<u32x2*>(ct + r * CROW + 2 * c) =
              u32x2{pack_bf16x2(a[4 * i], a[4 * i + 1]), pack_bf16x2(a[4 * i + 2], a[4 * i + 3])};
        }
    }
  }
  __syncthreads();
  {
    constexpr int CPR = BN / 8;          // 16-byte chunks per tile row
    constexpr int RPI = NT / CPR;        // rows per workgroup-wide store
    const int t = threadIdx.x;
    const int cc = t % CPR, r0 = t / CPR;
    const int gn = n0 + 8 * cc;
#pragma unroll 4
    for (int r = r0; r < BM; r += RPI) {
      const int gm = m0 + r;
      if (gm < M && gn < N)
        st128(C + (size_t)gm * N + gn, *reinterpret_cast<const u32x4*>(smem + r * CROW + 16 * cc));
    }
  }
}

template <int BM, int BN, bool GS>
static int launch(const void* A, const float* sA, const void* B, const float* sB, void* C, int M, int N, int K,
                  hipStream_t stream) {
  using CF = Cfg<BM, BN>;
  const long long tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7fffffffLL) return MX_ERR_SHAPE;
  const size_t smem = CF::LDS;
  constexpr auto kern = gemm_fp8_bs_kernel<BM, BN, GS>;
  MX_RETURN_IF_HIP(lds_limit_once<kern>((int)smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(NT), smem, stream, (const uint8_t*)A, sA, (const uint8_t*)B,
                     sB, (uint16_t*)C, M, N, K);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}


// ---------------------------------------------------------------------------
// Small M (decode batches) or few tiles: the product is a stream of the
// weights B, and 128x128 tiles would leave most CUs idle.
//  * A workgroup owns 32 columns x 32 MF rows of C, NW waves; wave w takes
//    the scale blocks kb = w, w + NW, ... of K, so every workgroup streams
//    its 32 columns of B once.  The row chunks of a column block and the
//    neighbouring column blocks run on one XCD, where they share B's
//    128-byte lines in L2.
//  * Each wave has a private ring of NSL slots, one scale block per slot:
//    A (32 MF rows x 128 B), B (128 k-rows x 32 B) and the block's scales
//    (one activation scale per row, the weight scale) by direct loads, so
//    one vmcnt wait lands all of them and no register is written behind
//    the compiler's back.  Slots are private, so the block loop has no
//    barrier; the wave issues block i+NSL-1 before it waits for block i.
//  * C^T = B^T . A^T on 32x32x64 fp8 MFMAs as in the main kernel: B^T
//    fragments by ds_read_b64_tr_b8 from 32-byte rows (eight rows fill the
//    256 banks' width, so a 32-lane phase is conflict free unswizzled), A^T
//    fragments by two ds_read_b128 from 128-byte rows whose chunk c sits at
//    c ^ ((m >> 1) & 7).  Two MFMAs build the block's partial, promoted with
//    one FMA per element: acc += (sA sB) * partial.
//  * The waves' accumulators meet in LDS at the end; wave i sums the four
//    result registers of every wave that hold n = 8i + 4(l/32) + {0..3}
//    and stores them (with 4 waves every register is summed once).
// ---------------------------------------------------------------------------
template <int MF, int NW, int NSL>
struct SmallCfg {
  static constexpr int A_B = 32 * MF * 128;   // A rows of one scale block
  static constexpr int B_B = 128 * 32;         // B k-rows of one scale block
  static constexpr int SA_OFF = A_B + B_B, SB_OFF = SA_OFF + 256;  // 64 row scales, 64 copies of sB
  static constexpr int SLOT = SB_OFF + 256;
  static constexpr int A_L = A_B / 1024, B_L = B_B / 1024;
  static constexpr int VM = A_L + B_L + 2;  // direct loads per block
  static constexpr int LDS = NW * NSL * SLOT;
  static_assert(NW == 4 || NW == 8, "waves");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert((NSL - 1) * VM < 64, "vmcnt range");
  static_assert(NW * MF * 64 * 16 * 4 <= LDS, "reduction area");
};

// f(integral_constant<int, I>) for I = 0 .. N-1, in order.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void unroll_n(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    unroll_n<N, I + 1>(f);
  }
}

__device__ __forceinline__ int swz_sa(int m) { return (m >> 1) & 7; }

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// As dma16 for 4 bytes per lane: lane i's dword lands at lds_addr + 4 i.
__device__ __forceinline__ void dma4(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, %0" ::"s"(sbase), "v"(voff), "s"(lds_addr)
               : "memory", "m0");
}
// s_waitcnt vmcnt(N) that also orders memory: no LDS read of the data it
// waits for is scheduled above it (this kernel has no barrier after it).
template <int N>
__device__ __forceinline__ void wait_vmcnt_mem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}
#pragma clang diagnostic pop

template <int MF, int NW, int NSL>
__global__ __launch_bounds__(64 * NW, 1) void gemm_fp8_bs_smallm_kernel(const uint8_t* __restrict__ A,
                                                                      const float* __restrict__ sA,
                                                                      const uint8_t* __restrict__ B,
                                                                      const float* __restrict__ sB,
                                                                      uint16_t* __restrict__ C, int M, int N,
                                                                      int K) {
  using CF = SmallCfg<MF, NW, NSL>;
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Workgroup -> (32-column block, chunk of 32 MF rows), the row chunks of a
  // column block adjacent: consecutive column blocks share 128-byte lines
  // of B, and one XCD (one L2) then fetches each line from HBM once.
  const int kblocks = K / SBK;
  const int nmc = (M + 32 * MF - 1) / (32 * MF);
  const int wid = xcd_remap(blockIdx.x, (int)gridDim.x);
  const int n0 = (wid / nmc) * 32, m0 = (wid % nmc) * 32 * MF;
  A += (size_t)m0 * K;
  sA += (size_t)m0 * kblocks;
  C += (size_t)m0 * N;
  M -= m0;  // rows of this chunk (more than 32 MF only past the last row read)
  const int nblocks_n = (N + 127) / 128;
  const int cnt = kblocks > wave ? (kblocks - wave + NW - 1) / NW : 0;  // this wave's blocks
  const uint32_t ring = lds_addr(smem) + wave * NSL * CF::SLOT;

  // Direct-load lane offsets.  A load n: rows 8n + l/8, LDS chunk l%8 taking
  // global chunk (l%8) ^ swz(row); B load n: k-rows 32n + l/2, chunk l%2
  // (columns past N re-read the last 16 valid ones; never stored).
  uint32_t a_off[CF::A_L], b_off[CF::B_L];
#pragma unroll
  for (int n = 0; n < CF::A_L; ++n) {
    const int row = 8 * n + (lane >> 3);
    a_off[n] = (uint32_t)min(row, M - 1) * (uint32_t)K + 16u * ((lane & 7) ^ swz_sa(row));
  }
#pragma unroll
  for (int n = 0; n < CF::B_L; ++n) {
    const int col = min(n0 + 16 * (lane & 1), N - 16) - n0;
    b_off[n] = (uint32_t)(32 * n + (lane >> 1)) * (uint32_t)N + col;
  }
  // scales: lane l loads the activation scale of row l (rows past M re-read
  // row M-1) and every lane the one weight scale of this column block
  const uint32_t sa_off = (uint32_t)min(lane, M - 1) * (uint32_t)kblocks * 4u;
  const uint32_t sb_off = (uint32_t)(n0 / 128) * 4u;
  // block i of this wave (kb = wave + NW i; past its last block, the last
  // one again, or block 0 for a wave without blocks) into slot I = i % NSL
  auto issue = [&](int i, auto slot_tag) {
    constexpr int I = decltype(slot_tag)::value;
    const int kb = cnt > 0 ? wave + NW * min(i, cnt - 1) : 0;
    const uint32_t st = ring + I * CF::SLOT;
#pragma unroll
    for (int n = 0; n < CF::A_L; ++n) dma16(A + (size_t)kb * SBK, a_off[n], st + n * 1024);
#pragma unroll
    for (int n = 0; n < CF::B_L; ++n) dma16(B + (size_t)kb * SBK * N + n0, b_off[n], st + CF::A_B + n * 1024);
    dma4(sA + kb, sa_off, st + CF::SA_OFF);
    dma4(sB + (size_t)kb * nblocks_n, sb_off, st + CF::SB_OFF);
  };

  // fragment lane addresses within a slot
  const int am = lane & 31, ah = lane >> 5;
  uint32_t a_col[2][2];  // [k step][16-byte half]
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int e = 0; e < 2; ++e) a_col[st][e] = am * 128 + 16 * ((4 * st + 2 * ah + e) ^ swz_sa(am));
  const int q = lane >> 4, jj = (lane & 15) >> 1, hh = lane & 1;
  const uint32_t b_col = CF::A_B + (32 * (q >> 1) + jj) * 32 + 16 * (q & 1) + 8 * hh;

  f32x16 acc[MF];
#pragma unroll
  for (int f = 0; f < MF; ++f) acc[f] = f32x16{};

  auto compute = [&](auto slot_tag) {
    constexpr int I = decltype(slot_tag)::value;
    const uint32_t st = ring + I * CF::SLOT;
    i32x8 bt[2], at[2][MF];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      u32x2 v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = lds_read_tr8_at(st + b_col + 64 * s2 * 32 + 8 * r * 32);
      bt[s2] = i32x8{(int)v[0][0], (int)v[0][1], (int)v[1][0], (int)v[1][1],
                     (int)v[2][0], (int)v[2][1], (int)v[3][0], (int)v[3][1]};
#pragma unroll
      for (int f = 0; f < MF; ++f) {
        const uint32_t r = st + 32 * f * 128;
        const u32x4 lo = lds_ld128(r + a_col[s2][0]);
        const u32x4 hi = lds_ld128(r + a_col[s2][1]);
        at[s2][f] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
    }
    const float sbv = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
        (uintptr_t)(st + CF::SB_OFF));
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      const float sav = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
          (uintptr_t)(st + CF::SA_OFF + 4 * (32 * f + am)));
      f32x16 p = mfma32_fp8(bt[0], at[0][f], f32x16{});
      p = mfma32_fp8(bt[1], at[1][f], p);
      acc[f] += (sav * sbv) * p;
    }
  };

  land_args(C);
  // prologue: blocks 0 .. NSL-2 in flight
  unroll_n<NSL - 1>([&](auto i_tag) { issue(decltype(i_tag)::value, i_tag); });

  // block i: issue block i + NSL - 1 into the slot block i - 1 used, then
  // wait for block i (the NSL - 1 blocks after it may be in flight)
  auto step = [&](int i, auto slot_tag) {
    constexpr int I = decltype(slot_tag)::value;
    // the previous block's fragment reads have completed before its slot
    // takes new data
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    issue(i + NSL - 1, std::integral_constant<int, (I + NSL - 1) % NSL>{});
    wait_vmcnt_mem<(NSL - 1) * CF::VM>();
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
  if (wave < 4) {
    const int gn = n0 + 8 * wave + 4 * ah;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] += red[((w * MF + f) * 16 + 4 * wave + j) * 64 + lane];
      const int gm = 32 * f + am;
      if (gm < M && gn < N)
        st64(C + (size_t)gm * N + gn, u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])});
    }
  }
}

template <int MF, int NW, int NSL>
static int launch_smallm(const void* A, const float* sA, const void* B, const float* sB, void* C, int M, int N, int K,
                         hipStream_t stream) {
  using CF = SmallCfg<MF, NW, NSL>;
  constexpr auto kern = gemm_fp8_bs_smallm_kernel<MF, NW, NSL>;
  MX_RETURN_IF_HIP(lds_limit_once<kern>(CF::LDS));
  const long long grid = (long long)((N + 31) / 32) * ((M + 32 * MF - 1) / (32 * MF));
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * NW), CF::LDS, stream, (const uint8_t*)A, sA,
                     (const uint8_t*)B, sB, (uint16_t*)C, M, N, K);
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
  // the activation-scale row offsets (row * K/128 * 4 bytes) are 32-bit
  if ((long long)M * (K / 128) * 4 > 0xffffffffLL) return MX_ERR_SHAPE;
  if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return MX_ERR_ALIGN;
  if (((uintptr_t)sA | (uintptr_t)sB) & 3) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const long long tiles256 = (long long)((M + 255) / 256) * ((N + 255) / 256);
  const long long tiles128 = (long long)((M + 127) / 128) * ((N + 127) / 128);
  // Rounds of 256 workgroups: a round of 256x256 tiles takes ~2.4 times a
  // round of 128x128 ones at the same K (measured 1.95-2.55 at 2048-3072),
  // so the big tile wins unless the small one needs fewer than 2.4 times
  // its rounds (3072^3: 1 round against 3, 57 vs 72 us; 2560^3: 1 against
  // 2, 44 vs 38 us).
  constexpr int SMALLM_NW = 4;  // waves of the weight-streaming kernel (each takes every 4th scale block)
  // Decode-sized M, or at most 64 tiles of 128x128 with M <= 512: stream
  // the weights with 32-column workgroups (graph-replayed: 256x4096x4096
  // 27.5 -> 22.5 us, 512x1024x4096 27.4 -> 12.3 us; 1024^3 stays tiled,
  // 10.6 against 11.8 us).
  if (M <= 32) return mx::gemm8::launch_smallm<1, SMALLM_NW, 4>(A, sA, B, sB, C, M, N, K, s);
  const long long tiles128s = (long long)((M + 127) / 128) * ((N + 127) / 128);
  if (M <= 64 || (tiles128s <= 64 && M <= 512))
    return mx::gemm8::launch_smallm<2, SMALLM_NW, 3>(A, sA, B, sB, C, M, N, K, s);
  const long long r256 = (tiles256 + 255) / 256, r128 = (tiles128 + 255) / 256;
  const bool big = tiles256 >= 256 || 12 * r256 < 5 * r128;
  // activation scales four blocks per 8-byte load when the blocks come in
  // fours and sA is 8-byte aligned (the interface asks only for 4)
  if (K % 512 == 0 && ((uintptr_t)sA & 7) == 0)
    return big ? mx::gemm8::launch<256, 256, true>(A, sA, B, sB, C, M, N, K, s)
               : mx::gemm8::launch<128, 128, true>(A, sA, B, sB, C, M, N, K, s);
  return big ? mx::gemm8::launch<256, 256, false>(A, sA, B, sB, C, M, N, K, s)
             : mx::gemm8::launch<128, 128, false>(A, sA, B, sB, C, M, N, K, s);
}
