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
//  * One workgroup = 4 waves = (up to 4 query heads sharing a KV head) x
//    (query sub-blocks).  K and V tiles of 64 keys are staged once in LDS
//    (double buffered, next tile's global loads in flight during the
//    current tile's MFMAs, one barrier per tile) and shared by the 4 waves.
//  * Softmax: the running max only moves when a lane's block max exceeds it
//    by more than 2^8 (lazy rescale, wave-uniform vote), the scale is folded
//    into the exp2 argument (one FMA + one exp2 per score), and the row sum
//    is accumulated with v_dot2 on the rounded P the PV MFMA consumes.
//  * Causal: workgroups launch heaviest-first; only diagonal / ragged tiles
//    are masked; tiles entirely above a wave's diagonal are skipped.
#include "mx_common.h"

// Query tiles (of 32) per wave.  1 keeps two waves per SIMD (the pair hides
// each other's softmax / LDS latency); 2 halves LDS reads per FLOP but needs
// about 512 registers and currently spills, so it is not the default.
#ifndef MX_GQA_QT
#define MX_GQA_QT 1
#endif

namespace mx {
namespace gqa {

constexpr int BN = 64;      // key/value positions per tile
constexpr int NWAVES = 4;
constexpr int NT = 64 * NWAVES;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;  // log2 headroom before the running max is raised

// LDS tiles are row-major copies of the K and V tiles ([BN keys][D]) with
// padded rows, so every fragment read of a lane is its base address plus a
// compile-time immediate and no read phase repeats a bank: K rows carry 16
// extra bytes (16-lane phases of 16-byte reads hit 16 distinct bank groups),
// V rows 64 (the 32-lane phases of the 8-byte transposing reads, 4 rows x 2
// column groups x 4 lanes, hit 32 distinct 8-byte slots).
template <int D>
struct Lds {
  static constexpr int K_ROW = D * 2 + 16;
  static constexpr int V_ROW = D * 2 + 64;
  static constexpr int K_BYTES = BN * K_ROW;
  static constexpr int V_BYTES = BN * V_ROW;
  static constexpr int STAGE = K_BYTES + V_BYTES;
  static constexpr int TOTAL = 2 * STAGE;
};

template <int D, typename T, bool CAUSAL, int QT>
__global__ __launch_bounds__(NT, QT == 1 ? 2 : 1) void gqa_fwd_kernel(const uint16_t* __restrict__ Q,
                                                                     const uint16_t* __restrict__ K,
                                                                     const uint16_t* __restrict__ V,
                                                                     uint16_t* __restrict__ O, int B, int Hq,
                                                                     int Hkv, int S, float sl2, int hpw) {
  constexpr int QW = 32 * QT;         // queries per wave
  constexpr int DC = D / 16;          // 16-deep k steps of QK^T
  constexpr int DT = D / 32;          // 32-row d tiles of O^T
  constexpr int K_LD = BN * D / 8 / NT;   // 16-B chunks of K (and of V) per thread
  static_assert(K_LD >= 1, "K tile split");
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5;      // lane half
  const int ql = lane & 31;     // query within a 32-query tile

  // ---- workgroup -> (qblock, b, kv head, head group) ----
  const int G = Hq / Hkv;
  const int qsb = NWAVES / hpw;            // query sub-blocks per workgroup
  const int QB = QW * qsb;                 // query rows per workgroup
  const int hgroups = G / hpw;
  const int nqb = (S + QB - 1) / QB;
  const int per_q = B * Hkv * hgroups;
  const int qb = nqb - 1 - (int)(blockIdx.x / per_q);  // heaviest first
  int rest = blockIdx.x % per_q;
  const int hg = rest % hgroups;
  rest /= hgroups;
  const int kvh = rest % Hkv;
  const int b = rest / Hkv;

  const int head = kvh * G + hg * hpw + (wave % hpw);
  const int q0w = qb * QB + (wave / hpw) * QW;   // this wave's first query
  const int q0wg = qb * QB;

  const size_t q_head = ((size_t)b * Hq + head) * S;
  const size_t kv_head = ((size_t)b * Hkv + kvh) * S;
  const uint16_t* Kh = K + kv_head * D;
  const uint16_t* Vh = V + kv_head * D;

  // ---- Q fragments (B operand of S^T = K Q^T), resident for the whole loop ----
  int qrow[QT];
  u32x4 qf[QT][DC];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    qrow[qt] = q0w + 32 * qt + ql;
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      const u32x4 x = ld128(Q + (q_head + min(qrow[qt], S - 1)) * D + dc * 16 + g * 8);
      qf[qt][dc] = (qrow[qt] < S) ? x : u32x4{0, 0, 0, 0};
    }
  }

  // ---- kv range ----
  const int kv_end_wg = CAUSAL ? min(S, q0wg + QB) : S;
  const int nblk = (kv_end_wg + BN - 1) / BN;
  const int kv_end_w = CAUSAL ? min(S, q0w + QW) : S;

  // ---- global -> register staging: K and V tiles row-major, 16-byte
  // chunks, chunk q = tid + i*NT -> row q / (D/8), chunk q % (D/8) ----
  constexpr int DB = D / 8;
  u32x4 rk[K_LD], rv[K_LD];

  auto load_kv = [&](int kv0) {
    if (kv0 + BN <= S) {  // uniform: every tile but a ragged last one
#pragma unroll
      for (int i = 0; i < K_LD; ++i) {
        const int q = tid + i * NT;
        const size_t off = (size_t)(kv0 + q / DB) * D + (q % DB) * 8;
        rk[i] = ld128(Kh + off);
        rv[i] = ld128(Vh + off);
      }
    } else {
      // rows past S are read from row S-1 (in bounds) and zeroed
#pragma unroll
      for (int i = 0; i < K_LD; ++i) {
        const int q = tid + i * NT;
        const int kv = kv0 + q / DB;
        const size_t off = (size_t)min(kv, S - 1) * D + (q % DB) * 8;
        const u32x4 xk = ld128(Kh + off), xv = ld128(Vh + off);
        rk[i] = (kv < S) ? xk : u32x4{0, 0, 0, 0};
        rv[i] = (kv < S) ? xv : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_kv = [&](int stage) {
    unsigned char* sk = smem + stage * Lds<D>::STAGE;
    unsigned char* sv = sk + Lds<D>::K_BYTES;
#pragma unroll
    for (int i = 0; i < K_LD; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<u32x4*>(sk + (q / DB) * Lds<D>::K_ROW + (q % DB) * 16) = rk[i];
      *reinterpret_cast<u32x4*>(sv + (q / DB) * Lds<D>::V_ROW + (q % DB) * 16) = rv[i];
    }
  };

  // Transposed V fragment addressing: lane (half g, sub-group sg, 4j+a)
  // reads key 16c + 8r + 4g + j at column 32dt + 16sg + 4a.
  const int v_sg = (lane >> 4) & 1, v_j = (lane >> 2) & 3, v_a = lane & 3;
  const int v_lane_off = (4 * g + v_j) * Lds<D>::V_ROW + (16 * v_sg + 4 * v_a) * 2;

  f32x16 acc_o[QT][DT];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int i = 0; i < DT; ++i) acc_o[qt][i] = f32x16{};
    m_run[qt] = -1e30f;
    l_run[qt] = 0.f;
  }

  if (nblk > 0) {
    load_kv(0);
    store_kv(0);
  }
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int cur = blk & 1;
    const int kv0 = blk * BN;
    if (blk + 1 < nblk) load_kv(kv0 + BN);

    if (kv0 < kv_end_w) {
      const unsigned char* sk = smem + cur * Lds<D>::STAGE;
      const unsigned char* sv = sk + Lds<D>::K_BYTES;

      // ---- S^T tiles: rows = keys (2 x 32), cols = queries (QT x 32) ----
      // 2*QT independent accumulator chains; each K fragment feeds QT
      // MFMAs and is read KLA k-steps ahead of its use.
      auto kread = [&](int t, int dc) {
        return *reinterpret_cast<const u32x4*>(sk + (t * 32 + ql) * Lds<D>::K_ROW + (dc * 2 + g) * 16);
      };
      f32x16 s[QT][2];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[qt][0] = s[qt][1] = f32x16{};
      constexpr int KLA = (QT == 1) ? 2 : 1;  // read lookahead (k-steps)
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
          for (int qt = 0; qt < QT; ++qt) s[qt][t] = mfma32<T>(kb[dc % (KLA + 1)][t], qf[qt][dc], s[qt][t]);
        __builtin_amdgcn_sched_barrier(0);  // keep the read lookahead
      }

      // V fragments of the first key chunk do not depend on the softmax:
      // issue them now so their latency hides under the VALU work below.
      auto vread = [&](int c, int dt) {
        const unsigned char* vb = sv + v_lane_off + (16 * c) * Lds<D>::V_ROW + dt * 64;
        const u32x2 lo = lds_read_tr16(vb);
        const u32x2 hi = lds_read_tr16(vb + 8 * Lds<D>::V_ROW);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vb[2][DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) vb[0][dt] = vread(0, dt);

      // ---- mask, online softmax (lane-local + one lane^32 exchange) ----
      // The running max m_run is kept in log2 units (scores * sl2) and is
      // only raised when some lane's block max exceeds it by more than
      // 2^kLazy: below that, p = 2^(s*sl2 - m_run) stays <= 2^kLazy and the
      // O/l rescale is skipped.  The decision is a wave-wide vote.
      const bool need_mask = (kv0 + BN > S) || (CAUSAL && kv0 + BN - 1 > q0w);
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        if (need_mask) {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int kv = kv0 + t * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
              const bool dead = (kv >= S) || (CAUSAL && kv > qrow[qt]);
              s[qt][t][e] = dead ? -INFINITY : s[qt][t][e];
            }
        }
        float mx = s[qt][0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[qt][t][e]);
        mx = max_xor32(mx) * sl2;
        if (__any(mx > m_run[qt] + kLazy)) {
          const float m_new = fmaxf(m_run[qt], mx);
          const float corr = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
          m_run[qt] = m_new;
          l_run[qt] *= corr;
#pragma unroll
          for (int i = 0; i < DT; ++i) acc_o[qt][i] *= corr;
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[qt][t][e] = __builtin_amdgcn_exp2f(fmaf(s[qt][t][e], sl2, -m_run[qt]));
      }

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
        }
        if (c + 1 < 4) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) vb[(c + 1) & 1][dt] = vread(c + 1, dt);
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) acc_o[qt][dt] = mfma32<T>(vb[c & 1][dt], pf[qt], acc_o[qt][dt]);
        __builtin_amdgcn_sched_barrier(0);  // keep the one-chunk read lookahead
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) l_run[qt] += lsum[qt];
    }

    if (blk + 1 < nblk) store_kv(cur ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane holds query qrow, d = 32dt + 8i + 4g + j ----
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l_tot = sum_xor32(l_run[qt]);
    const float inv = (l_tot > 0.f) ? 1.0f / l_tot : 0.f;
    if (qrow[qt] < S) {
      uint16_t* orow = O + (q_head + qrow[qt]) * D;
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
}

template <int D, typename T, bool CAUSAL, int QT>
static int launch(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, float scale,
                  hipStream_t stream) {
  const int G = Hq / Hkv;
  const int hpw = (G % 4 == 0) ? 4 : (G % 2 == 0 ? 2 : 1);
  const int QB = 32 * QT * (NWAVES / hpw);
  const long long grid = (long long)((S + QB - 1) / QB) * B * Hkv * (G / hpw);
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  auto kern = gqa_fwd_kernel<D, T, CAUSAL, QT>;
  MX_RETURN_IF_HIP(
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Lds<D>::TOTAL));
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NT), Lds<D>::TOTAL, stream, (const uint16_t*)Q,
                     (const uint16_t*)K, (const uint16_t*)V, (uint16_t*)O, B, Hq, Hkv, S, scale * kLog2e, hpw);
  MX_RETURN_IF_HIP(hipGetLastError());
  return MX_OK;
}

template <typename T, int QT>
static int dispatch(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, int D,
                    float scale, int causal, hipStream_t s) {
  if (D == 128) return causal ? launch<128, T, true, QT>(Q, K, V, O, B, Hq, Hkv, S, scale, s)
                              : launch<128, T, false, QT>(Q, K, V, O, B, Hq, Hkv, S, scale, s);
  if (D == 64) return causal ? launch<64, T, true, QT>(Q, K, V, O, B, Hq, Hkv, S, scale, s)
                             : launch<64, T, false, QT>(Q, K, V, O, B, Hq, Hkv, S, scale, s);
  return MX_ERR_UNSUPPORTED;
}

}  // namespace gqa
}  // namespace mx

extern "C" int mx_gqa_fwd(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S, int D,
                          float scale, int causal, int dtype, void* stream) {
  if (!Q || !K || !V || !O) return MX_ERR_NULL;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || Hq % Hkv) return MX_ERR_SHAPE;
  if (D != 64 && D != 128) return MX_ERR_SHAPE;
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return MX_ERR_SHAPE;
  if ((long long)B * Hq * S * D > (1LL << 40)) return MX_ERR_SHAPE;
  if (dtype != MX_DTYPE_BF16 && dtype != MX_DTYPE_F16) return MX_ERR_DTYPE;
  if (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V | (uintptr_t)O) & 15) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  constexpr int QT = MX_GQA_QT;
  if (dtype == MX_DTYPE_BF16) return mx::gqa::dispatch<mx::BF16, QT>(Q, K, V, O, B, Hq, Hkv, S, D, scale, causal, s);
  return mx::gqa::dispatch<mx::F16, QT>(Q, K, V, O, B, Hq, Hkv, S, D, scale, causal, s);
}
