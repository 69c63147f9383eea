// MLA absorbed (latent-cache) decode for gfx950.
//
//   O[b,h,:] = softmax_t( scale * Q[b,h,:] . KV[b,t,:] ) . KV[b,t,0:512]
//
// with Q[B,H,576], KV[B,T,576] (512 latent + 64 rope), O[B,H,512], bf16.
// This is softmax attention with one shared key/value head: the oracle is
// analysis/wave15-attention-architecture/reference/pytorch_reference_mla.py:66-81
// (`mla_naive`) with K := KV[b], V := KV[b][:, :512] broadcast to all heads,
// which is the weight-absorbed decode form of
// analysis/wave15-attention-research/MECHANISMS.md:91-94, 115-120.
//
// MI355X design.  With 128 heads the work sits near the HBM/MFMA ridge
// (about 240 flop per cache byte) and LDS fragment traffic is the tightest
// resource, so the two matrix products are partitioned differently across
// the 4 waves of a workgroup (one sequence, 128 heads, one slice of T):
//  * scores: wave g owns heads 32g..32g+31.  S^T = K . Q^T with 32x32x16
//    MFMAs, Q^T in VGPRs (36 k-steps), K fragments read from LDS; online
//    softmax with a lazily raised running max (the value accumulators are
//    rescaled only when a block max exceeds it by more than 2^16).  The
//    bf16 P^T fragments, already in MFMA B-operand layout, go to LDS (2 KB
//    per wave per stage);
//  * values: wave v owns latent columns 128v..128v+127 for all 128 heads:
//    O^T += V^T . P^T, where each V^T fragment (ds_read_b64_tr_b16 straight
//    from the row-major cache rows) serves the 4 head groups.  Per stage a
//    wave reads 8 KB of V and 8 KB of P instead of 32 KB of V;
//  * software pipeline: iteration i computes the scores of stage i, then
//    the values of stage i-1 with the softmax of stage i beside their
//    MFMAs (one barrier per stage);
//  * cache rows go HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging): latent rows into a 4-slot ring (a stage is read by the
//    scores of one iteration and the values of the next), rope rows into a
//    3-slot ring; 16-byte chunks are XOR-swizzled per row (swz_lat,
//    swz_rope below) so the K reads and the transposing V reads each hit
//    distinct bank slots;
//  * T is split across workgroups to fill the 256 CUs; each split writes
//    its normalised partial output (bf16, coalesced 512 B stores) and
//    (m, l) to the workspace, and a second kernel merges the splits with
//    the log-sum-exp rule.  With one split, O is written directly.
#include <type_traits>

#include "mx_common.h"

namespace mx {
namespace mla {

constexpr int DQK = 576;
constexpr int DV = 512;
constexpr int ROW_B = DQK * 2;          // 1152 bytes per cache row in HBM
constexpr int HPW = 32;                 // heads per score wave
constexpr int NWAVES = 4;
constexpr int NT = 64 * NWAVES;
constexpr int HPG = HPW * NWAVES;       // 128 heads per workgroup
constexpr int BT = 32;                  // tokens per stage
constexpr int KS = DQK / 16;            // 36 k-steps of S^T
constexpr int VT = DV / 32;             // 16 latent tiles of O^T
constexpr int VTW = VT / NWAVES;        // 4 latent tiles per value wave
constexpr int NLAT = 4;                 // latent ring slots (32 rows x 1 KB)
constexpr int NROPE = 3;                // rope ring slots (32 rows x 128 B)
constexpr int LPW = BT / NWAVES + 1;    // 1 KB loads per wave per stage (8 latent rows + 8 rope rows)
constexpr int LAT_B = BT * 1024;
constexpr int ROPE_B = BT * 128;
constexpr int ROPE_OFF = NLAT * LAT_B;                 // 131072
constexpr int P_OFF = ROPE_OFF + NROPE * ROPE_B;       // P^T fragments: [2 buf][4 group][2 k-half][64 lanes] x 16 B
constexpr int P_BUF = NWAVES * 2 * 64 * 16;
constexpr int C_OFF = P_OFF + 2 * P_BUF;               // rescale factors: [2 buf][4 group][32] fp32
constexpr int F_OFF = C_OFF + 2 * NWAVES * 32 * 4;     // rescale flags: [2 buf][4 group] int
constexpr int L_OFF = F_OFF + 2 * NWAVES * 4;          // final row sums: [4 group][32] fp32
constexpr int LDS_BYTES = L_OFF + NWAVES * 32 * 4;
constexpr int Q_WAVE_B = HPW * (1024 + 128);            // Q staging per wave (prologue only)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 16.0f;          // log2 headroom before a rescale
static_assert(BT * DQK / 8 == 64 * NWAVES * LPW, "a stage splits into whole wave loads");
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
static_assert(NWAVES * Q_WAVE_B <= LDS_BYTES, "Q staging fits the LDS allocation");
static_assert(DV / 16 == 32 && (DQK - DV) / 16 == 4, "Q fragment split: 32 latent + 4 rope k-steps");

// Chunk c of latent row t sits at chunk position c ^ swz_lat(t) of its
// 1024-byte row, chunk c of rope row t at c ^ swz_rope(t) of its 128-byte
// row.  LDS serves a 64-lane ds_read_b128 in four groups of 16 lanes, keyed
// by lane bit 5 and the parity of lane bits 2..4, and each group must hit
// 16 distinct 16-byte slots of the 256-byte bank window; a transposing
// ds_read_b64_tr_b16 is served in two 32-lane halves that must hit 32
// distinct 8-byte slots.
//  * K reads (lane l: token l%32, one chunk): the 16 tokens of a group are
//    {4a..4a+3} for four values of a with equal bit parity; swz_lat(t) =
//    (t%4)*4 + (t/4)%4 takes 16 distinct values over them.  Latent rows are
//    1024 B (every row starts at bank 0), so the slot is position % 16.
//    Rope rows are 128 B (two per window): swz_rope(t) = (t/2)%8 takes 8
//    distinct values over each parity of t in a group.
//  * V reads (a half-wave: 4 consecutive tokens 4a..4a+3 x one aligned quad
//    of 4 chunks): swz_lat's bits 2..3 are t%4, so the four rows land in
//    four different 64-byte quads; its bits 0..1 permute within a quad.
// swz_lat(t + 16) = swz_lat(t), so fragments 16 rows apart share lane
// offsets; rows 8 apart do not (they meet in one K read group).
__device__ __forceinline__ int swz_lat(int t) { return ((t & 3) << 2) | ((t >> 2) & 3); }
__device__ __forceinline__ int swz_rope(int t) { return (t >> 1) & 7; }

struct Split {
  int nsplit;
  int tps;  // tokens per split (multiple of the stage)
};

__host__ __device__ inline Split pick_split(int B, int H, int T) {
  const int hg = (H + HPG - 1) / HPG;
  const int nblk = (T + BT - 1) / BT;
  // Aim for >= 256 workgroups (one per CU) with at least 2 stages per split.
  int ns = 1;
  while ((long long)B * hg * ns < 256 && ns * 2 <= nblk / 2) ns *= 2;
  const int blocks_per = (nblk + ns - 1) / ns;
  Split s;
  s.nsplit = (nblk + blocks_per - 1) / blocks_per;
  s.tps = blocks_per * BT;
  return s;
}

// Stage i of a split: 32 latent rows of 1024 B (64 chunks) in latent slot
// i%4 and 32 rope rows of 128 B (8 chunks) in rope slot i%3, chunk c of row
// t at position c ^ swz_lat(t) (latent) or c ^ swz_rope(t) (rope).  Each
// 1 KB wave load fills one latent row (lane j <- chunk j ^ swz_lat(t), from
// a wave-uniform row address) or eight rope rows.  Rows past the end of the
// split re-read the last valid row (finite data whose scores are masked).
__device__ __forceinline__ void issue_part(const unsigned char* kvb, int tok0, int t1, uint32_t lat, uint32_t rope,
                                           int wave, int lane, int n) {
  constexpr int LR = BT / NWAVES;  // latent rows per wave
  if (n < LR) {
    uint32_t l16 = lane * 16;
    asm volatile("" : "+v"(l16));  // keep the per-row XOR here instead of a hoisted VGPR per row
    const int r = wave * LR + n;
    const int tok = min(tok0 + r, t1 - 1);
    dma16(kvb + (size_t)tok * ROW_B, l16 ^ (uint32_t)(16 * swz_lat(r)), lat + r * 1024);
  } else {
    const int r0 = wave * 8;
    const int tb = min(tok0 + r0, t1 - 1);
    const int tok = min(tok0 + r0 + (lane >> 3), t1 - 1);
    const uint32_t off = (uint32_t)(tok - tb) * ROW_B + 16 * (64 + ((lane & 7) ^ swz_rope(r0 + (lane >> 3))));
    dma16(kvb + (size_t)tb * ROW_B, off, rope + r0 * 128);
  }
}

// Partial tile of one (sequence, split, 32-head group): 64 slots (latent
// tile vt, row quad i) x 64 lanes x 4 bf16 = 32 KB, normalised by its own
// row sum; (m, l) per head in ws_ml.
constexpr int PT_U32 = VT * 4 * 64 * 2;  // uint32 words per partial tile

// Q is read as its latent part (512 values, rows q_ld elements apart) and
// its rope part (64 values at Qr, rows qr_ld apart): Qr = Q + 512 with
// q_ld = qr_ld = 576 for a packed [B,H,576] query.
__global__ __launch_bounds__(NT, 1) void mla_decode_kernel(const uint16_t* __restrict__ Q,
                                                          const uint16_t* __restrict__ Qr,
                                                          const uint16_t* __restrict__ KV,
                                                          uint16_t* __restrict__ O, uint32_t* __restrict__ ws_o,
                                                          float* __restrict__ ws_ml, int B, int H, int T,
                                                          float sl2, int nsplit, int tps, int q_ld, int qr_ld) {
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hsel = lane >> 5, l32 = lane & 31;

  const int HGB = (H + HPG - 1) / HPG;
  const int nwg = B * HGB * nsplit;
  const int id = xcd_remap(blockIdx.x, nwg);
  const int hgb = id % HGB;
  const int s = (id / HGB) % nsplit;
  const int b = id / (HGB * nsplit);

  const int t0 = s * tps;
  const int t1 = min(T, t0 + tps);
  const int nblk = (t1 - t0 + BT - 1) / BT;

  // Score role: heads hgb*128 + 32*wave + l32.  Padding heads (>= H) reuse
  // the last real head's row; their results are never stored.
  const unsigned char* kvb = reinterpret_cast<const unsigned char*>(KV + (size_t)b * T * DQK);
  const uint32_t lds0 = lds_addr(smem);

  // Q^T fragments of the wave's 32 heads.  The rows go HBM -> LDS with
  // direct loads, one 1 KB head row (latent part) or eight 128 B rope rows
  // per instruction, so every load is a contiguous run of the row; chunk c
  // of head h sits at position c ^ (h & 15) within its 256 B group (latent)
  // or c ^ ((h >> 1) & 7) (rope), which makes the fragment reads below
  // bank-conflict free.  Each wave stages into its own 36 KB, before the
  // cache ring starts.  Padding heads (>= H) read the last real head.
  u32x4 qf[KS];
  {
    const int h0 = hgb * HPG + wave * HPW;
    const int hb = min(h0, H - 1);
    const unsigned char* qb = reinterpret_cast<const unsigned char*>(Q + ((size_t)b * H + hb) * q_ld);
    const unsigned char* rb = reinterpret_cast<const unsigned char*>(Qr + ((size_t)b * H + hb) * qr_ld);
    const uint32_t qs = lds0 + wave * Q_WAVE_B;
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const int row = min(h0 + j, H - 1) - hb;
      const int c = (lane & ~15) | ((lane ^ j) & 15);
      dma16(qb, (uint32_t)row * q_ld * 2 + 16 * c, qs + j * 1024);
    }
#pragma unroll
    for (int j = 0; j < HPW / 8; ++j) {
      const int hl = 8 * j + (lane >> 3);
      const int row = min(h0 + hl, H - 1) - hb;
      const int c = (lane & 7) ^ ((hl >> 1) & 7);
      dma16(rb, (uint32_t)row * qr_ld * 2 + 16 * c, qs + HPW * 1024 + j * 1024);
    }
    wait_vmcnt<0>();  // this wave's rows landed; only this wave reads them
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = 2 * (ks & 31) + hsel;
      qf[ks] = ks < DV / 16 ? lds_ld128(qs + l32 * 1024 + 16 * ((c & ~15) | ((c ^ l32) & 15)))
                            : lds_ld128(qs + HPW * 1024 + l32 * 128 + 16 * ((c & 7) ^ ((l32 >> 1) & 7)));
    }
    __syncthreads();  // every wave holds its fragments before the ring overwrites the staging area
  }
  // part n (0..LPW-1) of this wave's direct loads of stage i
  auto issue_p = [&](int i, int n) {
    issue_part(kvb, t0 + i * BT, t1, lds0 + (i & (NLAT - 1)) * LAT_B, lds0 + ROPE_OFF + (i % NROPE) * ROPE_B, wave,
               lane, n);
  };
  auto issue = [&](int i) {
#pragma unroll
    for (int n = 0; n < LPW; ++n) issue_p(i, n);
  };
  land_args(O, ws_o, ws_ml);  // used only after the stage loop
  // Ring prologue.
  issue(0);
  if (nblk > 1) issue(1);

  // K fragment (A operand): row l32, chunk c = 2 ks + hsel at position
  // 16 (ks/8) + ((2 (ks%8) + hsel) ^ swz_lat(l32)): eight lane offsets plus
  // an immediate per k-step; the rope rows (ks >= 32, 128 B apart) have
  // four of their own.
  int koff[8], kroff[4];
#pragma unroll
  for (int m = 0; m < 8; ++m) koff[m] = l32 * 1024 + 16 * ((2 * m + hsel) ^ swz_lat(l32));
#pragma unroll
  for (int m = 0; m < 4; ++m) kroff[m] = l32 * 128 + 16 * ((2 * m + hsel) ^ swz_rope(l32));
  // V^T fragment via transposing reads: in lane group q = lane/16, lane
  // 4j + a addresses row 16 k2 + 4 (q>>1) + j + 8 h (h = 1 for the upper
  // half of k) and latent column 128 wave + 32 dt + 16 (q&1) + 4a, i.e.
  // chunk 16 wave + 4 dt + vw of that row: one lane offset per (dt, h).
  const int q4 = lane >> 4, ja = lane & 15;
  const int vj = ja >> 2, va = ja & 3;
  const int vrow = 4 * (q4 >> 1) + vj;
  const int vw = 2 * (q4 & 1) + (va >> 1);
  int v_off[VTW][2];
#pragma unroll
  for (int dt = 0; dt < VTW; ++dt)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      v_off[dt][h] = (vrow + 8 * h) * 1024 + 256 * wave + 8 * (va & 1) + 16 * ((4 * dt + vw) ^ swz_lat(vrow + 8 * h));

  // Value role accumulators: head group g, latent tile dt of this wave.
  f32x16 acc[NWAVES][VTW];
#pragma unroll
  for (int g = 0; g < NWAVES; ++g)
#pragma unroll
    for (int dt = 0; dt < VTW; ++dt) acc[g][dt] = f32x16{};
  float m_run = -1e30f, l_run = 0.f;

  // ---- S^T of stage si for head group `wave` (36 k-steps, one chain:
  // back-to-back accumulating MFMAs issue at the full rate).
  // With dma >= 0, this wave's direct loads of stage dma are issued one
  // per 4 k-steps, so they queue behind MFMAs instead of stalling the wave
  // at the address unit all at once. ----
  auto score_mfma = [&](int si, int dma) {
    const unsigned char* lat = smem + (si & (NLAT - 1)) * LAT_B;
    const unsigned char* rope = smem + ROPE_OFF + (si % NROPE) * ROPE_B;
    auto kread = [&](int ks) {
      return ks < 32 ? ld128(lat + koff[ks & 7] + 256 * (ks >> 3)) : ld128(rope + kroff[ks & 3]);
    };
    constexpr int KLA = 6;
    f32x16 sa = f32x16{};
    u32x4 kf[8];
#pragma unroll
    for (int ks = 0; ks < KLA; ++ks) kf[ks] = kread(ks);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + KLA < KS) kf[(ks + KLA) & 7] = kread(ks + KLA);
      sa = mfma32<BF16>(kf[ks & 7], qf[ks], sa);
      if ((ks & 3) == 2 && ks / 4 < LPW && dma >= 0) issue_p(dma, ks / 4);
      __builtin_amdgcn_sched_barrier(0);
    }
    return sa;
  };

  // Softmax pieces of stage si on its raw scores sc (lane holds head l32,
  // tokens tb + 8 i + 4 hsel + j for sc[4 i + j]).  The scale (log2 units)
  // is applied inside the exponent, exp2(s * sl2 - m): the row max of the
  // raw scores times sl2 > 0 is the max of the scaled ones, so no multiply
  // per score is needed before it.  Only the last stage of a slice can hold
  // tokens past its end: they are masked by one wave-uniform branch, not by
  // a select per score in every stage.
  auto mask_tail = [&](f32x16& sc, int si) {
    const int tb = t0 + si * BT;
    if (tb + BT > t1) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (tb + 8 * (r >> 2) + 4 * hsel + (r & 3) >= t1) sc[r] = -INFINITY;
    }
  };
  auto row_max = [&](const f32x16& sc, int r0, int r1, float& mx) {
#pragma unroll
    for (int r = r0; r < r1; ++r) mx = fmaxf(mx, sc[r]);
  };
  // Lazy running-max update; the rescale flag and factors of stage si go
  // to buffer si&1 for the value waves.
  auto update_max = [&](float mx, int si) {
    mx = max_xor32(mx) * sl2;  // raw -> log2 units
    int* flags = reinterpret_cast<int*>(smem + F_OFF) + (si & 1) * NWAVES;
    float* corrs = reinterpret_cast<float*>(smem + C_OFF) + ((si & 1) * NWAVES + wave) * 32;
    int flag = 0;
    if (__any(mx > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, mx);
      const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
      if (hsel == 0) corrs[l32] = corr;
      flag = si > 0;  // at stage 0 the value accumulators are still zero
    }
    if (lane == 0) flags[wave] = flag;
  };
  // P^T chunk k2 (bf16, B-operand layout, k order: tokens 4 hsel + j then
  // 8 + 4 hsel + j) of stage si to LDS, and its row sum.
  auto p_chunk = [&](const f32x16& sc, int si, int k2) {
    u32x4* pbuf = reinterpret_cast<u32x4*>(smem + P_OFF + (si & 1) * P_BUF);
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(fmaf(sc[8 * k2 + e], sl2, -m_run));
    const u32x4 pf{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                   pack_bf16x2(p[6], p[7])};
#pragma unroll
    for (int w = 0; w < 4; ++w) l_run = dot2_ones<BF16>(pf[w], l_run);
    pbuf[(wave * 2 + k2) * 64 + lane] = pf;
  };
  auto scores_alone = [&](int si, int dma) {
    f32x16 sc = score_mfma(si, dma);
    mask_tail(sc, si);
    float mx = -INFINITY;
    row_max(sc, 0, 16, mx);
    update_max(mx, si);
    p_chunk(sc, si, 0);
    p_chunk(sc, si, 1);
  };

  // ---- values of stage pi: O^T[128 wave + 32 dt .., heads] += V^T . P^T.
  // With SOFT, the softmax of stage pi+1 (scores sc, already masked) runs
  // beside the MFMAs: the row max beside the first k half, exp2 / P^T
  // beside the second. ----
  auto values = [&](int pi, auto with_soft, f32x16& sc) {
    constexpr bool SOFT = decltype(with_soft)::value;
    // all four flags in one LDS read (one wait instead of four)
    const u32x4 fl = *reinterpret_cast<const u32x4*>(smem + F_OFF + (pi & 1) * NWAVES * 4);
#pragma unroll
    for (int g = 0; g < NWAVES; ++g) {
      const int f = __builtin_amdgcn_readfirstlane(fl[g]);
      if (f) {
        const float c = reinterpret_cast<const float*>(smem + C_OFF)[((pi & 1) * NWAVES + g) * 32 + l32];
#pragma unroll
        for (int dt = 0; dt < VTW; ++dt) scale_acc(acc[g][dt], c);
      }
    }
    const unsigned char* lat = smem + (pi & (NLAT - 1)) * LAT_B;
    const u32x4* pbuf = reinterpret_cast<const u32x4*>(smem + P_OFF + (pi & 1) * P_BUF);
    // V^T fragments of both k halves are read up front (the second half's
    // reads overlap the first half's MFMAs).
    u32x4 vf[2][VTW];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < VTW; ++dt) {
        const unsigned char* p = lat + 16 * k2 * 1024;
        const u32x2 lo = lds_read_tr16(p + v_off[dt][0]);
        const u32x2 hi = lds_read_tr16(p + v_off[dt][1]);
        vf[k2][dt] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    float mx = -INFINITY;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      u32x4 pb[2];
      pb[0] = pbuf[k2 * 64 + lane];
#pragma unroll
      for (int g = 0; g < NWAVES; ++g) {
        if (g + 1 < NWAVES) pb[(g + 1) & 1] = pbuf[((g + 1) * 2 + k2) * 64 + lane];
#pragma unroll
        for (int dt = 0; dt < VTW; ++dt) acc[g][dt] = mfma32<BF16>(vf[k2][dt], pb[g & 1], acc[g][dt]);
        if constexpr (SOFT) {
          if (k2 == 0)
            row_max(sc, 4 * g, 4 * g + 4, mx);
          else if (g & 1)
            p_chunk(sc, pi + 1, g >> 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (SOFT) {
        if (k2 == 0) update_max(mx, pi + 1);
      }
    }
  };

  // Iteration i: scores of stage i (S^T MFMAs, with the direct loads of
  // stage i+2 spread among them), then the values of stage i-1 with the
  // softmax of stage i beside them.  Slot reuse: stage i+2 overwrites
  // latent slot (i+2)%4 (stage i-2, whose values finished before this
  // iteration's barrier) and rope slot (i+2)%3 (stage i-1, whose scores
  // did); the P^T/flag buffers alternate by stage.
  auto sync = [&](int i) {
    if (i + 1 < nblk)
      wait_vmcnt<LPW>();
    else
      wait_vmcnt<0>();
    __syncthreads();  // stage i landed for all waves; P^T of stage i-1 visible
  };
  sync(0);
  scores_alone(0, nblk > 2 ? 2 : -1);
  for (int i = 1; i < nblk; ++i) {
    sync(i);
    f32x16 sc = score_mfma(i, i + 2 < nblk ? i + 2 : -1);
    mask_tail(sc, i);
    values(i - 1, std::true_type{}, sc);
  }
  sync(nblk);
  {
    f32x16 none{};
    values(nblk - 1, std::false_type{}, none);
  }

  // Row sums to the value waves; (m, l) of each split to the workspace.
  const float l_tot = sum_xor32(l_run);
  float* lsum = reinterpret_cast<float*>(smem + L_OFF);
  if (hsel == 0) lsum[wave * 32 + l32] = l_tot;
  const int HW = (H + HPW - 1) / HPW;
  if (nsplit > 1 && hgb * NWAVES + wave < HW && hsel == 0) {
    float* pml = ws_ml + (((size_t)b * nsplit + s) * HW + hgb * NWAVES + wave) * 64 + 2 * l32;
    *reinterpret_cast<float2*>(pml) = float2{m_run, l_tot};
  }
  __syncthreads();

  // lane holds head hgb*128 + 32 g + l32, latent column 128 wave + 32 dt + 8 i + 4 hsel + j
#pragma unroll
  for (int g = 0; g < NWAVES; ++g) {
    const int hw = hgb * NWAVES + g;
    if (hw >= HW) break;  // the remaining head groups are all padding
    const float l = lsum[g * 32 + l32];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (nsplit == 1) {
      const int head = hw * HPW + l32;
      if (head < H) {
        uint16_t* orow = O + ((size_t)b * H + head) * DV + 128 * wave + 4 * hsel;
#pragma unroll
        for (int dt = 0; dt < VTW; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x16& a = acc[g][dt];
            st64(orow + 32 * dt + 8 * i, u32x2{pack_bf16x2(a[4 * i] * inv, a[4 * i + 1] * inv),
                                               pack_bf16x2(a[4 * i + 2] * inv, a[4 * i + 3] * inv)});
          }
      }
    } else {
      uint32_t* po = ws_o + (((size_t)b * nsplit + s) * HW + hw) * PT_U32;
#pragma unroll
      for (int dt = 0; dt < VTW; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x16& a = acc[g][dt];
          const int slot = (wave * VTW + dt) * 4 + i;
          st64(po + (slot * 64 + lane) * 2, u32x2{pack_bf16x2(a[4 * i] * inv, a[4 * i + 1] * inv),
                                                  pack_bf16x2(a[4 * i + 2] * inv, a[4 * i + 3] * inv)});
        }
    }
  }
}

// Merge the per-split softmax states:  o = sum_s w_s o_s / sum_s w_s,
// w_s = l_s 2^(m_s - max_s m_s), o_s the normalised split output.  An
// element-thread owns 16 bytes of a (b, 32-head group) partial tile: the
// adjacent lanes 2p, 2p+1 of one slot, i.e. 4 latent columns of two heads
// (2048 element-threads per tile), so the merge spreads over the whole GPU
// with 128-bit loads.  With many splits (small batches) SG threads share an
// element, each summing one of SG slices of the splits, and their sums meet
// in LDS: the serial chain of loads per thread stays near nsplit / SG.
// Merge workgroup sizes: 256 threads with one slice per element, 512 with
// split slices (measured: 512 took B4 H128 T4096 from 27.9 to 25.9 us; at
// one slice 256 measured 0.5-2 us faster than 512 at B16-B64).
constexpr int CMB_WG_ONE = 256, CMB_WG_MANY = 512;
constexpr int CMB_ET = VT * 4 * 32;  // element-threads per (b, 32-head group) tile = 2048

template <int SG>
struct CmbCfg {
  // Threads per workgroup: with split slices, larger workgroups cover more
  // output elements each, so fewer of them stage the same (m, l) pairs.
  static constexpr int WG = SG == 1 ? CMB_WG_ONE : CMB_WG_MANY;
  static constexpr int ET = WG / SG;         // element-threads per workgroup
  static constexpr int PER = CMB_ET / ET;    // workgroups per tile
  static constexpr int MAXS = SG == 1 ? 32 : 256;  // most splits; their (m, l) are staged in LDS (8 or 64 KB)
  static constexpr int MXS = WG / 16;        // slices of the splits in the per-head max
  static_assert(WG % 256 == 0 && WG <= 1024 && CMB_ET % ET == 0, "merge workgroup size");
};

template <int SG>
__global__ __launch_bounds__(CmbCfg<SG>::WG) void mla_combine_kernel(const uint32_t* __restrict__ ws_o,
                                                            const float* __restrict__ ws_ml,
                                                            uint16_t* __restrict__ O, int H, int nsplit) {
  using CF = CmbCfg<SG>;
  const int HW = (H + HPW - 1) / HPW;
  const int gi = blockIdx.x / CF::PER;          // b * HW + hw
  const int part = blockIdx.x % CF::PER;
  const int b = gi / HW, hw = gi % HW;
  const int sg = (int)threadIdx.x / CF::ET;     // split slice
  const int idx = part * CF::ET + (int)threadIdx.x % CF::ET;  // slot * 32 + lane pair
  const int lp = idx & 31, slot = idx >> 5;
  const int lane0 = 2 * lp;                     // lanes lane0, lane0 + 1
  const int l32 = lane0 & 31, hsel = lane0 >> 5;
  const size_t g0 = (size_t)b * nsplit * HW + hw;  // tile of split 0; split stride HW
  // The (m, l) pairs of the tile's 32 heads for every split (256 B per
  // split) are read once per workgroup into LDS, eight loads in flight per
  // thread; the host keeps nsplit <= MAXS.
  __shared__ f32x4 ml_lds[CF::MAXS * 16];
  __shared__ float2 mx_part[CF::MXS][16];  // [split residue mod MXS][head pair]: partial maxima
  const int n4 = nsplit * 16;
  for (int base = 0; base < n4; base += 8 * CF::WG) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * CF::WG + (int)threadIdx.x;
      if (i < n4) v[u] = *reinterpret_cast<const f32x4*>(ws_ml + (g0 + (size_t)(i >> 4) * HW) * 64 + 4 * (i & 15));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * CF::WG + (int)threadIdx.x;
      if (i < n4) ml_lds[i] = v[u];
    }
  }
  __syncthreads();
  {  // per-head maxima over the splits: MXS threads per head pair
    const int hp = threadIdx.x & 15, j = threadIdx.x >> 4;
    float2 m{-1e30f, -1e30f};
    for (int t = j; t < nsplit; t += CF::MXS) {
      const f32x4 x = ml_lds[t * 16 + hp];
      m.x = fmaxf(m.x, x[0]);
      m.y = fmaxf(m.y, x[2]);
    }
    mx_part[j][hp] = m;
  }
  __syncthreads();
  auto mlv_of = [&](int t) { return ml_lds[t * 16 + (l32 >> 1)]; };  // (m, l) of heads l32, l32 + 1 in split t
  float2 mmax{-1e30f, -1e30f};
#pragma unroll
  for (int j = 0; j < CF::MXS; ++j) {
    const float2 x = mx_part[j][l32 >> 1];
    mmax.x = fmaxf(mmax.x, x.x);
    mmax.y = fmaxf(mmax.y, x.y);
  }
  // this thread's slice of the splits
  const int s0 = (int)(((long long)nsplit * sg) / SG), s1 = (int)(((long long)nsplit * (sg + 1)) / SG);
  f32x4 o0{0.f, 0.f, 0.f, 0.f}, o1{0.f, 0.f, 0.f, 0.f};
  float l0 = 0.f, l1 = 0.f;
  const uint32_t* po = ws_o + g0 * PT_U32 + ((size_t)slot * 64 + lane0) * 2;
  const size_t sstride = (size_t)HW * PT_U32;
  auto acc1 = [&](const u32x4 p, const f32x4 mlv) {
    const float w0 = mlv[1] * __builtin_amdgcn_exp2f(mlv[0] - mmax.x);
    const float w1 = mlv[3] * __builtin_amdgcn_exp2f(mlv[2] - mmax.y);
    l0 += w0;
    l1 += w1;
    o0 += w0 * f32x4{bf16_bits_to_f32(p[0] & 0xffffu), bf16_bits_to_f32(p[0] >> 16),
                     bf16_bits_to_f32(p[1] & 0xffffu), bf16_bits_to_f32(p[1] >> 16)};
    o1 += w1 * f32x4{bf16_bits_to_f32(p[2] & 0xffffu), bf16_bits_to_f32(p[2] >> 16),
                     bf16_bits_to_f32(p[3] & 0xffffu), bf16_bits_to_f32(p[3] >> 16)};
  };
  // Eight splits per batch of loads: all independent, issued together.
  int s = s0;
  for (; s + 8 <= s1; s += 8) {
    u32x4 p[8];
    f32x4 mlv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      p[u] = ld128(po + (size_t)(s + u) * sstride);
      mlv[u] = mlv_of(s + u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc1(p[u], mlv[u]);
  }
  for (; s < s1; ++s) acc1(ld128(po + (size_t)s * sstride), mlv_of(s));
  if constexpr (SG > 1) {
    // the slices' sums meet in LDS (reusing the (m, l) staging area)
    __syncthreads();
    float* red = reinterpret_cast<float*>(ml_lds);  // [sg][10][ET]
    const int e = (int)threadIdx.x % CF::ET;
    const float v[10] = {o0[0], o0[1], o0[2], o0[3], o1[0], o1[1], o1[2], o1[3], l0, l1};
#pragma unroll
    for (int j = 0; j < 10; ++j) red[(sg * 10 + j) * CF::ET + e] = v[j];
    __syncthreads();
    if (sg != 0) return;
    float t[10];
#pragma unroll
    for (int j = 0; j < 10; ++j) {
      t[j] = 0.f;
#pragma unroll
      for (int g = 0; g < SG; ++g) t[j] += red[(g * 10 + j) * CF::ET + e];
    }
    o0 = f32x4{t[0], t[1], t[2], t[3]};
    o1 = f32x4{t[4], t[5], t[6], t[7]};
    l0 = t[8];
    l1 = t[9];
  }
  const int vt = slot >> 2, i = slot & 3;
  const int head0 = hw * HPW + l32;
  const float inv0 = l0 > 0.f ? 1.f / l0 : 0.f, inv1 = l1 > 0.f ? 1.f / l1 : 0.f;
  uint16_t* orow = O + ((size_t)b * H + head0) * DV + 32 * vt + 8 * i + 4 * hsel;
  if (head0 < H)
    st64(orow, u32x2{pack_bf16x2(o0[0] * inv0, o0[1] * inv0), pack_bf16x2(o0[2] * inv0, o0[3] * inv0)});
  if (head0 + 1 < H)
    st64(orow + DV, u32x2{pack_bf16x2(o1[0] * inv1, o1[1] * inv1), pack_bf16x2(o1[2] * inv1, o1[3] * inv1)});
}

// Split slices per merge element: about 32 splits per thread at most.
inline int combine_sg(int nsplit) { return nsplit >= 128 ? 8 : nsplit >= 64 ? 4 : nsplit >= 32 ? 2 : 1; }
inline int combine_max_splits(int nsplit) { return combine_sg(nsplit) == 1 ? CmbCfg<1>::MAXS : CmbCfg<8>::MAXS; }
inline int combine_per(int sg) {  // workgroups per (b, 32-head) tile
  return sg == 1 ? CmbCfg<1>::PER : sg == 2 ? CmbCfg<2>::PER : sg == 4 ? CmbCfg<4>::PER : CmbCfg<8>::PER;
}
inline long long combine_grid(int B, int HW, int nsplit) {
  return (long long)B * HW * combine_per(combine_sg(nsplit));
}

inline size_t workspace_bytes(int B, int H, int T) {
  const Split sp = pick_split(B, H, T);
  if (sp.nsplit <= 1) return 0;
  const size_t HW = (size_t)(H + HPW - 1) / HPW;
  return (size_t)B * sp.nsplit * HW * (PT_U32 * sizeof(uint32_t) + 2 * HPW * sizeof(float));
}

// Grid limits of the decode and combine launches.
static int check_grid(int B, int H, int T) {
  const Split sp = pick_split(B, H, T);
  const long long HGB = (H + HPG - 1) / HPG;
  const long long HW = (H + HPW - 1) / HPW;
  const long long grid = (long long)B * HGB * sp.nsplit;
  if (grid > 0x7fffffffLL || combine_grid(B, (int)HW, sp.nsplit) > 0x7fffffffLL) return MX_ERR_SHAPE;
  if (sp.nsplit > combine_max_splits(sp.nsplit)) return MX_ERR_SHAPE;  // pick_split keeps nsplit <= 256
  return MX_OK;
}

// The decode (+ combine) launches of one call; arguments (check_decode,
// check_grid) already checked.
static int launch_decode(const void* Q, const void* Qr, int q_ld, int qr_ld, const void* KV, void* O, int B, int H,
                         int T, float scale, void* workspace, hipStream_t s) {
  const Split sp = pick_split(B, H, T);
  const long long HGB = (H + HPG - 1) / HPG;
  const long long HW = (H + HPW - 1) / HPW;
  const long long grid = (long long)B * HGB * sp.nsplit;
  uint32_t* ws_o = (uint32_t*)workspace;
  float* ws_ml = sp.nsplit > 1 ? reinterpret_cast<float*>(ws_o + (size_t)B * sp.nsplit * HW * PT_U32) : nullptr;
  MX_RETURN_IF_HIP(lds_limit_once<mla_decode_kernel>(LDS_BYTES));
  hipLaunchKernelGGL(mla_decode_kernel, dim3((unsigned)grid), dim3(NT), LDS_BYTES, s, (const uint16_t*)Q,
                     (const uint16_t*)Qr, (const uint16_t*)KV, (uint16_t*)O, ws_o, ws_ml, B, H, T, scale * kLog2e,
                     sp.nsplit, sp.tps, q_ld, qr_ld);
  MX_RETURN_IF_HIP(hipGetLastError());
  if (sp.nsplit > 1) {
    const dim3 cg((unsigned)combine_grid(B, (int)HW, sp.nsplit));
    switch (combine_sg(sp.nsplit)) {
      case 1: hipLaunchKernelGGL(mla_combine_kernel<1>, cg, dim3(CmbCfg<1>::WG), 0, s, ws_o, ws_ml, (uint16_t*)O, H, sp.nsplit); break;
      case 2: hipLaunchKernelGGL(mla_combine_kernel<2>, cg, dim3(CmbCfg<2>::WG), 0, s, ws_o, ws_ml, (uint16_t*)O, H, sp.nsplit); break;
      case 4: hipLaunchKernelGGL(mla_combine_kernel<4>, cg, dim3(CmbCfg<4>::WG), 0, s, ws_o, ws_ml, (uint16_t*)O, H, sp.nsplit); break;
      default: hipLaunchKernelGGL(mla_combine_kernel<8>, cg, dim3(CmbCfg<8>::WG), 0, s, ws_o, ws_ml, (uint16_t*)O, H, sp.nsplit); break;
    }
    MX_RETURN_IF_HIP(hipGetLastError());
  }
  return MX_OK;
}

static int check_decode(const void* KV, int B, int H, int T, float scale) {
  if (B <= 0 || H <= 0 || T <= 0) return MX_ERR_SHAPE;
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return MX_ERR_SHAPE;
  if ((long long)B * T * DQK > (1LL << 40) || (long long)B * H > (1LL << 30)) return MX_ERR_SHAPE;
  if ((uintptr_t)KV & 15) return MX_ERR_ALIGN;
  return check_grid(B, H, T);
}

// Workspace of the absorbed step: q_lat [B,H,512] and o_lat [B,H,512] bf16,
// each rounded up to 256 bytes, then the decode's split partials.
inline size_t absorbed_workspace_bytes(int B, int H, int T) {
  const size_t lat = ((size_t)B * H * DV * 2 + 255) / 256 * 256;
  return 2 * lat + workspace_bytes(B, H, T);
}

}  // namespace mla
}  // namespace mx

extern "C" int mx_gemm_bf16_batched(const void* A, const void* B, void* C, int batch, int M, int N, int K, int lda,
                                    int ldb, int ldc, long long strideA, long long strideB, long long strideC,
                                    void* stream);
namespace mx {
namespace gemm {
int batched_check(const void* A, const void* B, void* C, int batch, int M, int N, int K, int lda, int ldb, int ldc,
                  long long strideA, long long strideB, long long strideC);
}  // namespace gemm
}  // namespace mx

extern "C" size_t mx_mla_decode_workspace(int B, int H, int T, int d_latent) {
  if (B <= 0 || H <= 0 || T <= 0 || d_latent != mx::mla::DV) return 0;
  return mx::mla::workspace_bytes(B, H, T);
}

extern "C" int mx_mla_decode_splits(int B, int H, int T) {
  if (B <= 0 || H <= 0 || T <= 0) return 0;
  return mx::mla::pick_split(B, H, T).nsplit;
}

extern "C" int mx_mla_decode(const void* Q, const void* KV, void* O, int B, int H, int T, int d_latent, int d_rope,
                             float scale, void* workspace, size_t ws_bytes, void* stream) {
  using namespace mx::mla;
  if (!Q || !KV || !O) return MX_ERR_NULL;
  if (B <= 0 || H <= 0 || T <= 0) return MX_ERR_SHAPE;
  if (d_latent != DV || d_rope != DQK - DV) return MX_ERR_UNSUPPORTED;
  if (const int e = check_decode(KV, B, H, T, scale)) return e;
  if (((uintptr_t)Q | (uintptr_t)O) & 15) return MX_ERR_ALIGN;
  const size_t need = workspace_bytes(B, H, T);
  if (need > 0 && (!workspace || ws_bytes < need)) return MX_ERR_WORKSPACE;
  if (need > 0 && ((uintptr_t)workspace & 15)) return MX_ERR_ALIGN;
  return launch_decode(Q, (const uint16_t*)Q + DV, DQK, DQK, KV, O, B, H, T, scale, workspace, (hipStream_t)stream);
}

extern "C" size_t mx_mla_decode_absorbed_workspace(int B, int H, int T) {
  if (B <= 0 || H <= 0 || T <= 0) return 0;
  return mx::mla::absorbed_workspace_bytes(B, H, T);
}

extern "C" int mx_mla_decode_absorbed(const void* q_nope, const void* q_rope, const void* KV, const void* w_uk,
                                      const void* w_uv, void* O, int B, int H, int T, int d_nope, int d_v,
                                      float scale, void* workspace, size_t ws_bytes, void* stream) {
  using namespace mx::mla;
  if (!q_nope || !q_rope || !KV || !w_uk || !w_uv || !O) return MX_ERR_NULL;
  if (const int e = check_decode(KV, B, H, T, scale)) return e;
  if (d_nope <= 0 || d_v <= 0 || (d_nope % 8) || (d_v % 8) || d_nope > 4096 || d_v > 4096) return MX_ERR_SHAPE;
  if (B > 65535 || H > 65535) return MX_ERR_SHAPE;
  if (((uintptr_t)q_nope | (uintptr_t)q_rope | (uintptr_t)w_uk | (uintptr_t)w_uv | (uintptr_t)O) & 15)
    return MX_ERR_ALIGN;
  const size_t need = absorbed_workspace_bytes(B, H, T);
  if (!workspace || ws_bytes < need) return MX_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const size_t lat = ((size_t)B * H * DV * 2 + 255) / 256 * 256;
  unsigned char* ws = (unsigned char*)workspace;
  void* q_lat = ws;
  void* o_lat = ws + lat;
  void* dws = workspace_bytes(B, H, T) ? (void*)(ws + 2 * lat) : nullptr;
  // Both products are checked before anything is enqueued.
  // q_lat[b,h,:] = q_nope[b,h,:] . W_UK[h]   (one product per head)
  const long long sq_uk = (long long)d_nope * DV, sq_uv = (long long)DV * d_v;
  if (const int e = mx::gemm::batched_check(q_nope, w_uk, q_lat, H, B, DV, d_nope, H * d_nope, DV, H * DV, d_nope,
                                            sq_uk, DV))
    return e;
  // o[b,h,:] = o_lat[b,h,:] . W_UV[h]
  if (const int e = mx::gemm::batched_check(o_lat, w_uv, O, H, B, d_v, DV, H * DV, d_v, H * d_v, DV, sq_uv, d_v))
    return e;
  int rc = mx_gemm_bf16_batched(q_nope, w_uk, q_lat, H, B, DV, d_nope, H * d_nope, DV, H * DV, d_nope, sq_uk, DV,
                                stream);
  if (rc) return rc;
  // latent attention with Q = [q_lat, q_rope]
  rc = launch_decode(q_lat, q_rope, DV, DQK - DV, KV, o_lat, B, H, T, scale, dws, s);
  if (rc) return rc;
  return mx_gemm_bf16_batched(o_lat, w_uv, O, H, B, d_v, DV, H * DV, d_v, H * d_v, DV, sq_uv, d_v, stream);
}
