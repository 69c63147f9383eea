// Fused grouped-query attention forward for gfx950 (flash-attention style).
//
// Semantics: cutile-attn-gqa/main.py:64-170 (one pass, online softmax in
// fp32, P cast to the I/O type before the PV product, final 1/l) and the
// oracle analysis/wave15-attention-architecture/reference/pytorch_reference.py:51-74,
// plus the causal mask this path adds.
//
// MI355X design:
//  * Scores are computed transposed, S^T = K · Q^T, with 32x32x16 MFMAs.
//    The query index then runs along lanes (lane l <-> query l%32 of a
//    32-query tile) and each lane holds 16 key positions per 32x32 tile, so
//    the softmax row max / row sum are lane-local plus one v_permlane32_swap.
//  * The probabilities never leave registers: the S^T accumulator of a
//    query tile is exactly the B operand (k = key, col = query) of
//    O^T = V^T · P^T.  The key order inside the registers is a fixed
//    permutation; V^T fragments are fetched in that order with gfx950's
//    transposing LDS read (ds_read_b64_tr_b16) from a row-major V tile, so
//    V is never transposed in registers.
//  * A wave owns QT tiles of 32 queries of one head; every K and V fragment
//    read from LDS feeds QT MFMAs, which is what bounds LDS traffic per FLOP.
//  * One workgroup = hpw query heads sharing a KV head x query sub-blocks:
//    QT = 1 runs 8 waves (two per SIMD, one workgroup per CU; 4 waves, two
//    workgroups per CU, for head dims whose stage does not split into 8
//    waves' loads), QT = 2 runs 4 waves (one per SIMD, 512 registers).  K
//    and V tiles of 64 keys are staged once in LDS (a 2- or 3-stage ring,
//    next tile's global loads in flight during the current tile's MFMAs,
//    one barrier per tile) and shared by all waves.  The workgroup's query
//    rows per head (the tile's BLOCK_M) are waves x 32 QT / hpw; hpw is a
//    launch argument, so every BLOCK_M with hpw | G is the same kernel.
//  * Softmax: the running max only moves when a lane's block max exceeds it
//    by more than 2^8 (lazy rescale, wave-uniform vote).  The scale, in log2
//    units, is folded into Q once in the prologue, so the score MFMAs return
//    log2-domain scores and each score costs one exp2; the row sum is
//    accumulated with v_dot2 on the rounded P the PV MFMA consumes.
//  * Causal: each workgroup takes a heavy and a light query block (block p
//    and its mirror nqb-1-p), so all workgroups carry the same number of
//    key tiles and finish together; only diagonal / ragged tiles are
//    masked; tiles entirely above a wave's diagonal are skipped.
#include <type_traits>

#include "mx_common.h"

namespace mx {
namespace gqa {

constexpr int BN = 64;      // key/value positions per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;  // log2 headroom before the running max is raised

// Chunk positions inside LDS rows (16-byte chunk c of row r): K rows hold
// chunk c at c ^ kswz(r), V rows at c ^ vswz(r).  The LDS serves 256 B per
// clock (64 banks); a 16-byte read phase is 16 lanes, an 8-byte phase 32.
//  * K fragment reads: 16 lanes read one chunk of 16 consecutive rows, so
//    kswz spreads those rows over 16 distinct 16-byte slots (mod 256 B):
//    r&15 for 256-byte rows; (r>>1)&7 for 128- and 384-byte rows (rows start
//    at two bank phases, 0 and 128 B); (r>>2)&3 for 192-byte rows (four
//    phases, 0/192/128/64 B).  The XOR only flips low chunk bits, so a chunk
//    stays inside its row.
//  * transposing V reads: 32 lanes read 4 consecutive rows x one aligned
//    quad of chunks (64 B), so vswz gives each of the 4 rows its own quad:
//    (r&3)<<2 for 256-byte rows, ((r>>1)&1)<<2 for 128-byte rows.  Rows 8
//    and 16 apart share the swizzle, so fragment offsets stay immediates.
template <int ROW>
__device__ __forceinline__ int kswz(int r) {
  if constexpr (ROW == 256) return r & 15;
  else if constexpr (ROW == 192) return (r >> 2) & 3;
  else return (r >> 1) & 7;
}
template <int ROW>
__device__ __forceinline__ int vswz(int r) {
  return ROW == 256 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2);
}

// One stage = K tile [BN keys][DQK] then V tile [BN keys][DV], unpadded
// swizzled rows.  Direct load n of a stage fills bytes 1024n .. 1024n+1023
// of the stage (K tile first), whatever rows that spans.
template <int DQK, int DV, int NWAVES>
struct Lds {
  static constexpr int ROWK = DQK * 2, ROWV = DV * 2;
  static constexpr int TILEK = BN * ROWK, TILEV = BN * ROWV;
  static constexpr int STAGE = TILEK + TILEV;
  static constexpr int NLK = TILEK / 1024;           // direct loads per K tile
  static constexpr int LPW = STAGE / 1024 / NWAVES;  // direct loads per wave per stage
  static_assert(TILEK % 1024 == 0 && TILEV % 1024 == 0 && STAGE % (1024 * NWAVES) == 0, "whole loads per wave");
  static_assert((ROWK == 128 || ROWK == 192 || ROWK == 256 || ROWK == 384) && (ROWV == 128 || ROWV == 256),
                "row sizes with a conflict-free swizzle");
};

// Waves per workgroup: 8 (two per SIMD, one workgroup per CU) when a stage
// splits into whole 1 KB loads for 8 waves, else 4 (two workgroups per CU).
// With 8, twice the queries share every K/V tile staged in LDS.
template <int DQK, int DV>
constexpr int waves_for() {
  return ((DQK + DV) * 2 * BN / 1024) % 8 == 0 ? 8 : 4;
}

template <int QT>
struct Ring {
  static constexpr int NS = QT == 1 ? 2 : 3;  // stages (QT=1 keeps two waves per SIMD)
};

// Waves of a workgroup for the default kernel of a head-dim pair (QT = 1).
template <int DQK, int DV>
constexpr int default_waves() {
  return waves_for<DQK, DV>();
}

template <int DQK, int DV, typename T, bool CAUSAL, int QT, int NWAVES>
__global__ __launch_bounds__(64 * NWAVES, QT == 1 ? 2 : 1) void gqa_fwd_kernel(const uint16_t* __restrict__ Q,
                                                                     const uint16_t* __restrict__ K,
                                                                     const uint16_t* __restrict__ V,
                                                                     uint16_t* __restrict__ O, int B, int Hq,
                                                                     int Hkv, int S, float sl2, int hpw) {
  constexpr int QW = 32 * QT;         // queries per wave
  constexpr int DC = DQK / 16;        // 16-deep k steps of QK^T
  constexpr int DT = DV / 32;         // 32-row d tiles of O^T
  constexpr int NS = Ring<QT>::NS;
  using L = Lds<DQK, DV, NWAVES>;
  extern __shared__ __align__(1024) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;      // lane half
  const int ql = lane & 31;     // query within a 32-query tile

  // ---- workgroup -> (qblock, b, kv head, head group) ----
  const int G = Hq / Hkv;
  const int qsb = NWAVES / hpw;            // query sub-blocks per workgroup
  const int QB = QW * qsb;                 // query rows per workgroup
  const int hgroups = G / hpw;
  const int nqb = (S + QB - 1) / QB;
  const int per_q = B * Hkv * hgroups;
  // Causal: workgroup p takes query block nqb-1-p, then its mirror p, so
  // every workgroup carries about the same number of key tiles.
  const int p = (int)(blockIdx.x / per_q);
  const int nrep = (CAUSAL && nqb - 1 - p != p) ? 2 : 1;
  int rest = blockIdx.x % per_q;
  const int hg = rest % hgroups;
  rest /= hgroups;
  const int kvh = rest % Hkv;
  const int b = rest / Hkv;

  const int head = kvh * G + hg * hpw + (wave % hpw);
  const size_t q_head = ((size_t)b * Hq + head) * S;
  const size_t kv_head = ((size_t)b * Hkv + kvh) * S;
  const unsigned char* Kh = reinterpret_cast<const unsigned char*>(K + kv_head * DQK);
  const unsigned char* Vh = reinterpret_cast<const unsigned char*>(V + kv_head * DV);

  for (int rep = 0; rep < nrep; ++rep) {
  const int qb = CAUSAL ? (rep == 0 ? nqb - 1 - p : p) : p;
  const int q0w = qb * QB + (wave / hpw) * QW;   // this wave's first query
  const int q0wg = qb * QB;

  // ---- Q fragments (B operand of S^T = K Q^T), resident for the whole loop.
  // Rows past S read row S-1; their outputs are never stored. ----
  int qrow[QT];
  u32x4 qf[QT][DC];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    qrow[qt] = q0w + 32 * qt + ql;
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      // Fold the softmax scale (in log2 units) into Q once, so the score
      // MFMAs produce log2-domain scores directly.
      const u32x4 x = ld128(Q + (q_head + min(qrow[qt], S - 1)) * DQK + dc * 16 + g * 8);
      u32x4 y;
#pragma unroll
      for (int w = 0; w < 4; ++w) y[w] = T::pack2(T::to_f32(x[w] & 0xffffu) * sl2, T::to_f32(x[w] >> 16) * sl2);
      qf[qt][dc] = y;
    }
  }

  // ---- kv range ----
  const int kv_end_wg = CAUSAL ? min(S, q0wg + QB) : S;
  const int nblk = (kv_end_wg + BN - 1) / BN;
  const int kv_end_w = CAUSAL ? min(S, q0w + QW) : S;

  // ---- HBM -> LDS with direct loads: wave load ld of a stage fills stage
  // bytes 1024ld .. +1023 (the K tile, then the V tile); lane i takes byte
  // 16i of it, i.e. row r = byte / ROW, chunk c = (byte % ROW) / 16, stored
  // at chunk position c ^ k/vswz(r).  Rows past S re-read row S-1 (finite
  // data that the mask or a zero P cancels). ----
  const uint32_t lds0 = lds_addr(smem);
  auto ld_row = [&](int ld) {
    const bool vt = ld >= L::NLK;
    return (1024 * (vt ? ld - L::NLK : ld) + 16 * lane) / (vt ? L::ROWV : L::ROWK);
  };
  auto ld_chunk = [&](int ld) {  // swizzled byte offset of this lane's chunk inside its row
    const bool vt = ld >= L::NLK;
    const int byte = 1024 * (vt ? ld - L::NLK : ld) + 16 * lane;
    const int r = byte / (vt ? L::ROWV : L::ROWK), c = (byte % (vt ? L::ROWV : L::ROWK)) / 16;
    return 16 * (c ^ (vt ? vswz<L::ROWV>(r) : kswz<L::ROWK>(r)));
  };
  // Lane offsets of the wave's loads relative to the tile's first row, so a
  // full tile needs no VALU work: a scalar row base plus these.
  uint32_t ld_off[L::LPW];
#pragma unroll
  for (int n = 0; n < L::LPW; ++n) {
    const int ld = wave * L::LPW + n;
    ld_off[n] = (uint32_t)ld_row(ld) * (ld >= L::NLK ? L::ROWV : L::ROWK) + ld_chunk(ld);
  }
  // load n of tile blk, rows past S-1 clamped to S-1 (no branch: it can sit
  // between the MFMAs of a k step)
  auto issue_part = [&](int blk, int n) {
    const int ld = wave * L::LPW + n;
    const bool vt = ld >= L::NLK;
    const int kv = min(blk * BN + ld_row(ld), S - 1);
    dma16(vt ? Vh : Kh, (uint32_t)kv * (vt ? L::ROWV : L::ROWK) + ld_chunk(ld),
          lds0 + (blk % NS) * L::STAGE + ld * 1024);
  };
  auto issue = [&](int blk) {
    const int kv0 = blk * BN;
    const uint32_t st = lds0 + (blk % NS) * L::STAGE;
    if (kv0 + BN <= S) {
#pragma unroll
      for (int n = 0; n < L::LPW; ++n) {
        const int ld = wave * L::LPW + n;
        const bool vt = ld >= L::NLK;
        dma16((vt ? Vh + (size_t)kv0 * L::ROWV : Kh + (size_t)kv0 * L::ROWK), ld_off[n], st + ld * 1024);
      }
    } else {
#pragma unroll
      for (int n = 0; n < L::LPW; ++n) {
        const int ld = wave * L::LPW + n;
        const bool vt = ld >= L::NLK;
        const int kv = min(kv0 + ld_row(ld), S - 1);
        dma16(vt ? Vh : Kh, (uint32_t)kv * (vt ? L::ROWV : L::ROWK) + ld_chunk(ld), st + ld * 1024);
      }
    }
  };
  if (rep > 0) __syncthreads();  // every wave is done with the previous block's ring
  land_args(O);  // O is used only after the tile loop
  issue(0);
  wait_vmcnt<0>();  // the Q loads and stage 0 complete together
#pragma unroll
  for (int p = 1; p < NS - 1; ++p)
    if (p < nblk) issue(p);

  // K fragment (A operand of S^T): key row 32t + ql, chunk 2dc + g at
  // position (2dc + g) ^ kswz(ql): one lane offset per dc, t an immediate.
  uint32_t koff[DC];  // absolute LDS addresses in stage 0
#pragma unroll
  for (int dc = 0; dc < DC; ++dc) koff[dc] = lds0 + ql * L::ROWK + 16 * ((2 * dc + g) ^ kswz<L::ROWK>(ql));
  // Transposed V fragment: lane (half g, sub-group sg, 4j+a) reads key
  // 16c + 8r + 4g + j at column 32dt + 16sg + 4a, i.e. chunk 4dt + 2sg +
  // a/2 of a row whose swizzle is vswz(4g + j): one lane offset per dt.
  const int v_sg = (lane >> 4) & 1, v_j = (lane >> 2) & 3, v_a = lane & 3;
  const int vrow = 4 * g + v_j;
  const int vw = 2 * v_sg + (v_a >> 1);
  uint32_t v_off[DT];  // absolute LDS addresses in stage 0
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    v_off[dt] = lds0 + L::TILEK + vrow * L::ROWV + 16 * ((4 * dt + vw) ^ vswz<L::ROWV>(vrow)) + 8 * (v_a & 1);

  // Softmax state per query (log2 units).  The score MFMAs start from
  // neg_m = -m_run instead of zero, so they return s - m_run directly.
  f32x16 acc_o[QT][DT];
  float m_run[QT], l_run[QT];
  f32x16 neg_m[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int i = 0; i < DT; ++i) acc_o[qt][i] = f32x16{};
    m_run[qt] = 0.f;
    l_run[qt] = 0.f;
    neg_m[qt] = f32x16{};
  }

  // One key tile; STG = blk % NS is a compile-time constant so every LDS
  // fragment address is a lane offset plus an immediate.
  auto tile = [&](int blk, auto stg_tag) {
    constexpr int STG = decltype(stg_tag)::value;
    // stage blk landed (this wave's loads), then visible to all waves;
    // the stage read in iteration blk-1 is free for stage blk+NS-1.
    if constexpr (NS == 3) {
      if (blk + 1 < nblk)
        wait_vmcnt<L::LPW>();
      else
        wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    // the next tile's loads go out one per k step of the S^T MFMAs below
    // rather than all at once, which queues every wave's loads behind the
    // barrier
    const bool load_next = blk + NS - 1 < nblk;
    const int kv0 = blk * BN;
    // a wave that skips this tile still issues its share of the next one
    if (kv0 >= kv_end_w && load_next) issue(blk + NS - 1);

    if (kv0 < kv_end_w) {
      constexpr uint32_t st = STG * L::STAGE;

      // ---- S^T tiles: rows = keys (2 x 32), cols = queries (QT x 32) ----
      // 2*QT independent accumulator chains; each K fragment feeds QT
      // MFMAs and is read KLA k-steps ahead of its use.
      auto kread = [&](int t, int dc) {
        return lds_ld128(koff[dc] + st + t * 32 * L::ROWK);
      };
      f32x16 s[QT][2];
      // Start value of the score chains.  With QT = 2 it is rebuilt from
      // m_run for every tile instead of holding 32 registers across the loop.
      auto start_m = [&](int qt) {
        if constexpr (QT == 1) {
          return neg_m[qt];
        } else {
          f32x16 v;
#pragma unroll
          for (int e = 0; e < 16; ++e) v[e] = -m_run[qt];
          return v;
        }
      };
      // Wave priority: the two waves sharing a SIMD issue their MFMA phases
      // ahead of the other's softmax VALU work, which then fills the gaps.
      __builtin_amdgcn_s_setprio(1);
      constexpr int KLA = DQK > 128 ? 1 : 2;  // read lookahead (k-steps); 1 keeps the 192-wide Q in registers
      u32x4 kb[KLA + 1][2];
#pragma unroll
      for (int i = 0; i < KLA; ++i) {
        kb[i][0] = kread(0, i);
        kb[i][1] = kread(1, i);
      }
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        if (dc + KLA < DC) {
          kb[(dc + KLA) % (KLA + 1)][0] = kread(0, dc + KLA);
          kb[(dc + KLA) % (KLA + 1)][1] = kread(1, dc + KLA);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
            s[qt][t] = mfma32<T>(kb[dc % (KLA + 1)][t], qf[qt][dc], dc == 0 ? start_m(qt) : s[qt][t]);
#pragma unroll
        for (int n = 0; n < L::LPW; ++n)
          if (dc == n * DC / L::LPW && load_next) issue_part(blk + NS - 1, n);
        __builtin_amdgcn_sched_barrier(0);  // keep the read lookahead
      }

      // V fragments of the first key chunk do not depend on the softmax:
      // issue them now so their latency hides under the VALU work below.
      auto vread = [&](int c, int dt) {
        const uint32_t vb = v_off[dt] + st + (16 * c) * L::ROWV;
        const u32x2 lo = lds_read_tr16_at(vb);
        const u32x2 hi = lds_read_tr16_at(vb + 8 * L::ROWV);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vb[2][DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) vb[0][dt] = vread(0, dt);

      __builtin_amdgcn_s_setprio(0);
      // ---- mask, online softmax (lane-local + one lane^32 exchange) ----
      // s holds s - m_run (log2 units).  The running max is set from the
      // first tile and afterwards only raised when some lane's block max
      // exceeds it by more than 2^kLazy: below that, p = 2^(s - m_run)
      // stays <= 2^kLazy and neither O, l nor the scores are touched.  The
      // decision is a wave-wide vote.
      const bool need_mask = (kv0 + BN > S) || (CAUSAL && kv0 + BN - 1 > q0w);
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        if (need_mask) {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int kv = kv0 + t * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
              const bool dead = (kv >= S) | (CAUSAL & (kv > qrow[qt]));
              s[qt][t][e] = dead ? -INFINITY : s[qt][t][e];
            }
        }
        float mx = s[qt][0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[qt][t][e]);
        mx = max_xor32(mx);
        const bool first = blk == 0;  // every wave processes tile 0
        if (first || __any(mx > kLazy)) {
          // first tile: the max itself; later: only upward moves
          const float shift = first ? mx : fmaxf(mx, 0.f);
          const float corr = __builtin_amdgcn_exp2f(-shift);
          m_run[qt] += shift;
          l_run[qt] *= corr;
#pragma unroll
          for (int i = 0; i < DT; ++i) {
            if constexpr (QT == 1) {
              acc_o[qt][i] *= corr;
            } else {
              agpr_settle(acc_o[qt][i]);
              scale_acc(acc_o[qt][i], corr);
              agpr_settle(acc_o[qt][i]);  // before the next asm MFMA reads it
            }
          }
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[qt][t][e] -= shift;
#pragma unroll
          for (int e = 0; e < 16; ++e) neg_m[qt][e] = QT == 1 ? -m_run[qt] : 0.f;
        }
        // exp2 of key chunk 0 now; chunk c+1 is exponentiated inside the
        // P.V step of chunk c, in the shadow of its MFMAs.
#pragma unroll
        for (int e = 0; e < 8; ++e) s[qt][0][e] = __builtin_amdgcn_exp2f(s[qt][0][e]);
      }

      __builtin_amdgcn_s_setprio(1);
      // ---- O^T += V^T P^T over 4 key chunks of 16 ----
      float lsum[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) lsum[qt] = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int t = c >> 1, i0 = 2 * (c & 1);
        // P^T operand: keys 16c + 4g + {0..3} then 16c + 8 + 4g + {0..3}
        u32x4 pf[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const f32x16& x = s[qt][t];
          pf[qt] = u32x4{T::pack2(x[4 * i0 + 0], x[4 * i0 + 1]), T::pack2(x[4 * i0 + 2], x[4 * i0 + 3]),
                         T::pack2(x[4 * i0 + 4], x[4 * i0 + 5]), T::pack2(x[4 * i0 + 6], x[4 * i0 + 7])};
          // the row sum uses the rounded P the MFMA consumes
#pragma unroll
          for (int w = 0; w < 4; ++w) lsum[qt] = dot2_ones<T>(pf[qt][w], lsum[qt]);
          if constexpr (QT != 1) operand_settle(pf[qt]);  // read by asm MFMAs
        }
        if (c + 1 < 4) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) vb[(c + 1) & 1][dt] = vread(c + 1, dt);
          const int t1 = (c + 1) >> 1, j1 = 8 * ((c + 1) & 1);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int e = 0; e < 8; ++e) s[qt][t1][j1 + e] = __builtin_amdgcn_exp2f(s[qt][t1][j1 + e]);
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            // QT = 2: O^T stays in AGPRs (see mfma32_agpr)
            if constexpr (QT == 1)
              acc_o[qt][dt] = mfma32<T>(vb[c & 1][dt], pf[qt], acc_o[qt][dt]);
            else
              mfma32_agpr<T>(acc_o[qt][dt], vb[c & 1][dt], pf[qt]);
          }
        if (c + 1 < 4) {
          // packs of chunk c first, then each MFMA followed by its share of
          // chunk c+1's exp2, the next chunk's V reads and the row sums
          // (QT = 2's asm MFMAs are in no group; the compiler places them,
          // which measured faster than one scheduling region per MFMA)
          __builtin_amdgcn_sched_group_barrier(0x002, 4 * QT, 0);
#pragma unroll
          for (int m = 0; m < DT * QT; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x400, 8 * QT / (DT * QT), 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * DT / (DT * QT), 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4 * QT / (DT * QT), 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the one-chunk read lookahead
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) l_run[qt] += lsum[qt];
      __builtin_amdgcn_s_setprio(0);
    }
  };
  for (int blk = 0; blk < nblk; blk += NS) {
    tile(blk, std::integral_constant<int, 0>{});
    if (blk + 1 < nblk) tile(blk + 1, std::integral_constant<int, 1>{});
    if constexpr (NS == 3)
      if (blk + 2 < nblk) tile(blk + 2, std::integral_constant<int, 2>{});
  }

  // ---- normalise and store: lane holds query qrow, d = 32dt + 8i + 4g + j ----
  if constexpr (QT != 1) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) agpr_settle(acc_o[qt][dt]);
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l_tot = sum_xor32(l_run[qt]);
    const float inv = (l_tot > 0.f) ? 1.0f / l_tot : 0.f;
    if (qrow[qt] < S) {
      uint16_t* orow = O + (q_head + qrow[qt]) * DV;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = dt * 32 + 8 * i + 4 * g;
          const f32x16& a = acc_o[qt][dt];
          st64(orow + d, u32x2{T::pack2(a[4 * i] * inv, a[4 * i + 1] * inv),
                               T::pack2(a[4 * i + 2] * inv, a[4 * i + 3] * inv)});
        }
    }
  }
}  // q-block loop
}

template <int DQK, int DV, typename T, bool CAUSAL, int QT, int NWAVES>
static int launch(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, float scale,
                  int hpw, hipStream_t stream) {
  const int G = Hq / Hkv;
  const int QB = 32 * QT * (NWAVES / hpw);
  const int nqb = (S + QB - 1) / QB;
  const long long grid = (long long)(CAUSAL ? (nqb + 1) / 2 : nqb) * B * Hkv * (G / hpw);
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  constexpr auto kern = gqa_fwd_kernel<DQK, DV, T, CAUSAL, QT, NWAVES>;
  constexpr int lds = Ring<QT>::NS * Lds<DQK, DV, NWAVES>::STAGE;
  MX_RETURN_IF_HIP(lds_limit_once<kern>(lds));
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * NWAVES), lds, stream, (const uint16_t*)Q, (const uint16_t*)K,
                     (const uint16_t*)V, (uint16_t*)O, B, Hq, Hkv, S, scale * kLog2e, hpw);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

// A GQA launch shape: the kernel variant (queries per wave = 32 QT, waves
// per workgroup) and hpw heads of one KV group per workgroup.  Kernel
// variants: (QT 1, 8 waves) two waves per SIMD and one workgroup per CU;
// (QT 1, 4 waves) two workgroups per CU; (QT 2, 4 waves) one wave per SIMD
// with 512 registers, where each K and V fragment feeds two MFMAs.
struct Tile {
  int qt, nwaves, hpw;
};

// Heads per workgroup of the default tile: as many heads of a KV group as
// divide G, up to 4 (with 8 waves, each K/V tile then serves 256 queries).
inline int default_hpw(int G) { return (G % 4 == 0) ? 4 : (G % 2 == 0 ? 2 : 1); }

// The launch of a tile (BLOCK_M query rows of a head per workgroup,
// BLOCK_N keys per LDS stage, wave_m query rows per wave), or
// MX_ERR_UNSUPPORTED when no kernel of this library has it.  BLOCK_N is the
// kernels' 64-key stage.  wave_m 32 takes the 8-wave kernel when hpw =
// 256 / BLOCK_M divides G, else the 4-wave one (hpw = 128 / BLOCK_M); wave_m
// 64 the QT = 2 kernel (hpw = 256 / BLOCK_M).  GQA head dims 64 and 128.
inline int tile_for(int G, int D, int block_m, int block_n, int wave_m, Tile* t) {
  if (block_n != BN || block_m <= 0 || (D != 64 && D != 128)) return MX_ERR_UNSUPPORTED;
  auto fits = [&](int qt, int nwaves) {
    const int rows = nwaves * 32 * qt;  // query rows of a workgroup, over all its heads
    if (rows % block_m) return false;
    const int hpw = rows / block_m;
    if (hpw > nwaves || nwaves % hpw || G % hpw) return false;
    *t = Tile{qt, nwaves, hpw};
    return true;
  };
  if (wave_m == 32) return fits(1, 8) || fits(1, 4) ? MX_OK : MX_ERR_UNSUPPORTED;
  if (wave_m == 64) return fits(2, 4) ? MX_OK : MX_ERR_UNSUPPORTED;
  return MX_ERR_UNSUPPORTED;
}

template <int D, typename T, bool CAUSAL>
static int launch_tile(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S,
                       float scale, const Tile& t, hipStream_t s) {
  if (t.qt == 2) return launch<D, D, T, CAUSAL, 2, 4>(Q, K, V, O, B, Hq, Hkv, S, scale, t.hpw, s);
  if (t.nwaves == 4) return launch<D, D, T, CAUSAL, 1, 4>(Q, K, V, O, B, Hq, Hkv, S, scale, t.hpw, s);
  return launch<D, D, T, CAUSAL, 1, 8>(Q, K, V, O, B, Hq, Hkv, S, scale, t.hpw, s);
}

template <typename T>
static int dispatch_tile(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, int D,
                         float scale, int causal, const Tile& t, hipStream_t s) {
  if (D == 128)
    return causal ? launch_tile<128, T, true>(Q, K, V, O, B, Hq, Hkv, S, scale, t, s)
                  : launch_tile<128, T, false>(Q, K, V, O, B, Hq, Hkv, S, scale, t, s);
  return causal ? launch_tile<64, T, true>(Q, K, V, O, B, Hq, Hkv, S, scale, t, s)
                : launch_tile<64, T, false>(Q, K, V, O, B, Hq, Hkv, S, scale, t, s);
}

template <int DQK, int DV, typename T>
static int launch_default(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S,
                          float scale, int causal, hipStream_t s) {
  constexpr int NW = default_waves<DQK, DV>();
  const int hpw = default_hpw(Hq / Hkv);
  return causal ? launch<DQK, DV, T, true, 1, NW>(Q, K, V, O, B, Hq, Hkv, S, scale, hpw, s)
                : launch<DQK, DV, T, false, 1, NW>(Q, K, V, O, B, Hq, Hkv, S, scale, hpw, s);
}

// (qk head dim, v head dim) pairs with a kernel: the GQA head dims 64 and
// 128, and the MLA prefill pairs 192/128 (DeepSeek-V3: 128 nope + 64 rope,
// v 128) and 96/64 (the reference's correctness shape).
template <typename T>
static int dispatch(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, int dqk,
                    int dv, float scale, int causal, hipStream_t s) {
  if (dqk == 128 && dv == 128) return launch_default<128, 128, T>(Q, K, V, O, B, Hq, Hkv, S, scale, causal, s);
  if (dqk == 64 && dv == 64) return launch_default<64, 64, T>(Q, K, V, O, B, Hq, Hkv, S, scale, causal, s);
  if (dqk == 192 && dv == 128) return launch_default<192, 128, T>(Q, K, V, O, B, Hq, Hkv, S, scale, causal, s);
  if (dqk == 96 && dv == 64) return launch_default<96, 64, T>(Q, K, V, O, B, Hq, Hkv, S, scale, causal, s);
  return MX_ERR_UNSUPPORTED;
}

static int check_args(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, int dqk,
                      float scale, int dtype) {
  if (!Q || !K || !V || !O) return MX_ERR_NULL;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || Hq % Hkv) return MX_ERR_SHAPE;
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return MX_ERR_SHAPE;
  if ((long long)B * Hq * S * dqk > (1LL << 40)) return MX_ERR_SHAPE;
  if (dtype != MX_DTYPE_BF16 && dtype != MX_DTYPE_F16) return MX_ERR_DTYPE;
  if (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V | (uintptr_t)O) & 15) return MX_ERR_ALIGN;
  return MX_OK;
}

}  // namespace gqa
}  // namespace mx

extern "C" int mx_gqa_fwd(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, int D,
                          float scale, int causal, int dtype, void* stream) {
  if (D != 64 && D != 128) return (!Q || !K || !V || !O) ? MX_ERR_NULL : MX_ERR_SHAPE;
  if (const int e = mx::gqa::check_args(Q, K, V, O, B, Hq, Hkv, S, D, scale, dtype)) return e;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MX_DTYPE_BF16) return mx::gqa::dispatch<mx::BF16>(Q, K, V, O, B, Hq, Hkv, S, D, D, scale, causal, s);
  return mx::gqa::dispatch<mx::F16>(Q, K, V, O, B, Hq, Hkv, S, D, D, scale, causal, s);
}

extern "C" int mx_gqa_fwd_tile_check(int Hq, int Hkv, int D, int block_m, int block_n, int wave_m) {
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || (D != 64 && D != 128)) return MX_ERR_SHAPE;
  mx::gqa::Tile t;
  return mx::gqa::tile_for(Hq / Hkv, D, block_m, block_n, wave_m, &t);
}

extern "C" int mx_gqa_fwd_default_block_m(int Hq, int Hkv, int D) {
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || (D != 64 && D != 128)) return MX_ERR_SHAPE;
  return 8 * 32 / mx::gqa::default_hpw(Hq / Hkv);
}

extern "C" int mx_gqa_fwd_tile(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S,
                               int D, float scale, int causal, int dtype, int block_m, int block_n, int wave_m,
                               void* stream) {
  if (D != 64 && D != 128) return (!Q || !K || !V || !O) ? MX_ERR_NULL : MX_ERR_SHAPE;
  if (const int e = mx::gqa::check_args(Q, K, V, O, B, Hq, Hkv, S, D, scale, dtype)) return e;
  mx::gqa::Tile t;
  if (const int e = mx::gqa::tile_for(Hq / Hkv, D, block_m, block_n, wave_m, &t)) return e;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MX_DTYPE_BF16)
    return mx::gqa::dispatch_tile<mx::BF16>(Q, K, V, O, B, Hq, Hkv, S, D, scale, causal, t, s);
  return mx::gqa::dispatch_tile<mx::F16>(Q, K, V, O, B, Hq, Hkv, S, D, scale, causal, t, s);
}

namespace mx {
namespace gqa {
template <int D, typename T, bool C>
static const void* tile_kernel(const Tile& t) {
  if (t.qt == 2) return reinterpret_cast<const void*>(gqa_fwd_kernel<D, D, T, C, 2, 4>);
  if (t.nwaves == 4) return reinterpret_cast<const void*>(gqa_fwd_kernel<D, D, T, C, 1, 4>);
  return reinterpret_cast<const void*>(gqa_fwd_kernel<D, D, T, C, 1, 8>);
}
template <int D, typename T>
static const void* tile_kernel_c(const Tile& t, int causal) {
  return causal ? tile_kernel<D, T, true>(t) : tile_kernel<D, T, false>(t);
}
}  // namespace gqa
}  // namespace mx

// Registers and scratch (spill) bytes per lane of the kernel a tile runs:
// what the reference's block sweep reads from its compiled kernels.
extern "C" int mx_gqa_fwd_tile_info(int Hq, int Hkv, int D, int dtype, int causal, int block_m, int block_n,
                                    int wave_m, int* vgprs, int* scratch_bytes) {
  if (!vgprs || !scratch_bytes) return MX_ERR_NULL;
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || (D != 64 && D != 128)) return MX_ERR_SHAPE;
  if (dtype != MX_DTYPE_BF16 && dtype != MX_DTYPE_F16) return MX_ERR_DTYPE;
  mx::gqa::Tile t;
  if (const int e = mx::gqa::tile_for(Hq / Hkv, D, block_m, block_n, wave_m, &t)) return e;
  using mx::gqa::tile_kernel_c;
  const void* f = D == 128 ? (dtype == MX_DTYPE_BF16 ? tile_kernel_c<128, mx::BF16>(t, causal)
                                                    : tile_kernel_c<128, mx::F16>(t, causal))
                           : (dtype == MX_DTYPE_BF16 ? tile_kernel_c<64, mx::BF16>(t, causal)
                                                    : tile_kernel_c<64, mx::F16>(t, causal));
  hipFuncAttributes a{};
  MX_RETURN_IF_HIP(hipFuncGetAttributes(&a, f));
  *vgprs = a.numRegs;
  *scratch_bytes = (int)a.localSizeBytes;
  return MX_OK;
}

extern "C" int mx_mla_prefill_fwd(const void* Q, const void* K, const void* V, void* O, int B, int H, int S, int d_qk,
                                  int d_v, float scale, int causal, int dtype, void* stream) {
  if (const int e = mx::gqa::check_args(Q, K, V, O, B, H, H, S, d_qk, scale, dtype)) return e;
  if (!((d_qk == 192 && d_v == 128) || (d_qk == 96 && d_v == 64) || (d_qk == 128 && d_v == 128) ||
        (d_qk == 64 && d_v == 64)))
    return MX_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MX_DTYPE_BF16)
    return mx::gqa::dispatch<mx::BF16>(Q, K, V, O, B, H, H, S, d_qk, d_v, scale, causal, s);
  return mx::gqa::dispatch<mx::F16>(Q, K, V, O, B, H, H, S, d_qk, d_v, scale, causal, s);
}
