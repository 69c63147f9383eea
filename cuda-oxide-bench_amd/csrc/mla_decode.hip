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
// MI355X design.  With 128 heads the work is close to the HBM/MFMA ridge
// (about 240 flop per cache byte), so both the single read of the cache and
// the matrix-core rate matter:
//  * a wave owns 32 heads and 32 tokens of each stage and runs 32x32x16
//    MFMAs: S^T = K . Q^T (Q^T for its heads stays in VGPRs, 36 k-steps),
//    then O^T += V^T . P^T with P^T straight from the score registers and
//    V^T read from the row-major cache tile with ds_read_b64_tr_b16;
//  * a workgroup (4 waves) owns one sequence, one slice of T ("split") and
//    NHG head groups; the NTP = 4/NHG waves of one head group take
//    different tokens of each stage and are merged at the end;
//  * cache rows go HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging) into a ring of stages, 147 KB in all; the 16-byte chunks of
//    a row are XOR-swizzled inside groups of 8 so that both the K reads
//    (8 consecutive tokens, one chunk) and the transposing V reads (4
//    consecutive tokens, two chunks) hit distinct banks;
//  * the running max is raised lazily (only when a block max exceeds it by
//    more than 2^8), so the 256-register O accumulator is rarely rescaled;
//  * T is split across workgroups to fill the 256 CUs; each split writes
//    (m, l, unnormalised o) to the workspace in a lane-major layout (1 KB
//    coalesced stores) and a second kernel merges the splits with the
//    log-sum-exp rule.  With one split, O is written directly.
#include "mx_common.h"

namespace mx {
namespace mla {

constexpr int DQK = 576;
constexpr int DV = 512;
constexpr int CH = DQK / 8;             // 72 sixteen-byte chunks per cache row
constexpr int ROW_B = DQK * 2;          // 1152 bytes per cache row in LDS
constexpr int HPW = 32;                 // heads per wave
constexpr int TPW = 32;                 // tokens per wave per stage
constexpr int NWAVES = 4;
constexpr int NT = 64 * NWAVES;
constexpr int KS = DQK / 16;            // 36 k-steps of S^T
constexpr int VT = DV / 32;             // 16 dv tiles of O^T
constexpr int LDS_BYTES = NWAVES * TPW * ROW_B;  // 147456
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;           // log2 headroom before a rescale

template <int NTP>
struct Cfg {
  static constexpr int NHG = NWAVES / NTP;              // head groups per workgroup
  static constexpr int HPG = NHG * HPW;                 // heads per workgroup
  static constexpr int BT = NTP * TPW;                  // tokens per stage
  static constexpr int STAGE_B = BT * ROW_B;
  static constexpr int NS = LDS_BYTES / STAGE_B;        // ring depth
  static constexpr int LPW = BT / NWAVES + NTP;         // 1 KB loads per wave per stage
  static_assert(BT * CH == 64 * NWAVES * LPW, "stage splits into whole wave loads");
  static_assert(NS >= 2, "double buffering at least");
};

// Chunk c of row t sits at chunk position c ^ swz(t) of its row.  swz maps
// t%8 to 0,2,4,6,1,3,5,7: distinct over 8 rows (K reads: 8 consecutive
// tokens, one chunk) and with distinct halves over each aligned group of 4
// rows (transposing V reads: 4 consecutive tokens, two adjacent chunks), so
// both read patterns are bank-conflict free on 1024 B and 128 B rows.
__device__ __forceinline__ int swz(int t) { return ((t & 3) << 1) | ((t >> 2) & 1); }

// acc *= c for an accumulator held in AGPRs: read, multiply, write back one
// register at a time (VALU cannot read AGPRs), without ever materialising
// the whole tile in VGPRs.
__device__ __forceinline__ void scale_acc(f32x16& acc, float c) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float x = acc[e], t;
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(t)
                 : "v"(c));
    acc[e] = x;
  }
}

struct Split {
  int nsplit;
  int tps;  // tokens per split (multiple of the stage)
};

template <int NTP>
__host__ __device__ inline Split pick_split(int B, int H, int T) {
  using C = Cfg<NTP>;
  const int hg = (H + C::HPG - 1) / C::HPG;
  const int nblk = (T + C::BT - 1) / C::BT;
  // Aim for >= 256 workgroups (one per CU) with at least 2 stages per split.
  int ns = 1;
  while ((long long)B * hg * ns < 256 && ns * 2 <= nblk / 2) ns *= 2;
  const int blocks_per = (nblk + ns - 1) / ns;
  Split s;
  s.nsplit = (nblk + blocks_per - 1) / blocks_per;
  s.tps = blocks_per * C::BT;
  return s;
}

// Stage layout in LDS: BT latent rows of 1024 B (64 chunks), then BT rope
// rows of 128 B (8 chunks), chunk c of row t at position c ^ swz(t).
// Issue the direct loads of one stage: each 1 KB wave load fills one latent
// row (lane i <- chunk i ^ swz(t), from a wave-uniform row address) or
// eight rope rows.  Rows past the end of the split re-read the last valid
// row (finite data whose scores are masked).
template <int NTP>
__device__ __forceinline__ void issue_stage(const unsigned char* kvb, int tok0, int t1, uint32_t stage, int wave,
                                            int lane) {
  using C = Cfg<NTP>;
  constexpr int LR = C::BT / NWAVES;  // latent rows per wave
  uint32_t l16 = lane * 16;
  asm volatile("" : "+v"(l16));  // keep the per-row XORs in the loop instead of 8 hoisted VGPRs
#pragma unroll
  for (int n = 0; n < LR; ++n) {
    const int r = wave * LR + n;
    const int tok = min(tok0 + r, t1 - 1);
    dma16(kvb + (size_t)tok * ROW_B, l16 ^ (uint32_t)(16 * swz(r)), stage + r * 1024);
  }
  const bool full = tok0 + C::BT <= t1;
#pragma unroll
  for (int n = 0; n < NTP; ++n) {
    const int r0 = (wave * NTP + n) * 8;
    const int tb = min(tok0 + r0, t1 - 1);
    int tok = tok0 + r0 + (lane >> 3);
    if (!full) tok = min(tok, t1 - 1);
    const uint32_t off = (uint32_t)(tok - tb) * ROW_B + 16 * (64 + ((lane & 7) ^ swz(lane >> 3)));
    dma16(kvb + (size_t)tb * ROW_B, off, stage + C::BT * 1024 + r0 * 128);
  }
}

// Wait until at most `ahead` stages of this wave's loads are outstanding.
template <int LPW, int NS>
__device__ __forceinline__ void wait_stages(int ahead) {
  if constexpr (NS >= 4) {
    if (ahead >= 2) {
      wait_vmcnt<2 * LPW>();
      return;
    }
  }
  if constexpr (NS >= 3) {
    if (ahead >= 1) {
      wait_vmcnt<LPW>();
      return;
    }
  }
  wait_vmcnt<0>();
}

template <int NTP>
__global__ __launch_bounds__(NT, 1) void mla_decode_kernel(const uint16_t* __restrict__ Q,
                                                          const uint16_t* __restrict__ KV,
                                                          uint16_t* __restrict__ O, float* __restrict__ ws_o,
                                                          float* __restrict__ ws_ml, int B, int H, int T,
                                                          float sl2, int nsplit, int tps) {
  using C = Cfg<NTP>;
  extern __shared__ __align__(1024) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hgi = wave % C::NHG;  // head group of this wave
  const int tp = wave / C::NHG;   // token part of each stage
  const int hsel = lane >> 5, l32 = lane & 31;

  const int HGB = (H + C::HPG - 1) / C::HPG;
  const int nwg = B * HGB * nsplit;
  const int id = xcd_remap(blockIdx.x, nwg);
  const int hgb = id % HGB;
  const int s = (id / HGB) % nsplit;
  const int b = id / (HGB * nsplit);

  const int hw = hgb * C::NHG + hgi;  // 32-head group index
  const int head = hw * HPW + l32;
  const bool head_ok = head < H;
  const int t0 = s * tps;
  const int t1 = min(T, t0 + tps);
  const int nblk = (t1 - t0 + C::BT - 1) / C::BT;

  // Q^T fragments (B operand): lane holds head `head`, features 16 ks + 8 hsel .. +7.
  // Padding heads (head >= H) reuse the last real head's row; their
  // results are never stored.
  u32x4 qf[KS];
  {
    const uint16_t* qrow = Q + ((size_t)b * H + min(head, H - 1)) * DQK + 8 * hsel;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = ld128(qrow + 16 * ks);
  }

  // Ring prologue.  The Q loads are completed together with stage 0, so no
  // compiler-visible load is outstanding once the cache loads stream.
  const unsigned char* kvb = reinterpret_cast<const unsigned char*>(KV + (size_t)b * T * DQK);
  const uint32_t lds0 = lds_addr(smem);
  issue_stage<NTP>(kvb, t0, t1, lds0, wave, lane);
  wait_vmcnt<0>();
#pragma unroll
  for (int p = 1; p < C::NS - 1; ++p)
    if (p < nblk) issue_stage<NTP>(kvb, t0 + p * C::BT, t1, lds0 + p * C::STAGE_B, wave, lane);

  // K fragment (A operand): row tp*32 + l32, chunk 2 ks + hsel.
  const int krow = tp * TPW + l32;
  const int kx = swz(krow);
  const int k_lat = krow * 1024;
  const int k_rope = C::BT * 1024 + krow * 128;
  auto kread = [&](const unsigned char* st, int ks) {
    const int c = 2 * ks + hsel;
    return ks < 32 ? ld128(st + k_lat + 16 * (c ^ kx)) : ld128(st + k_rope + 16 * ((c - 64) ^ kx));
  };
  // V^T fragment via transposing reads: in lane group q = lane/16, lane
  // 4j + a addresses row tp*32 + 16 k2 + 4 (q>>1) + j (+8 for the upper
  // half of k) and dv 32 vt + 16 (q&1) + 4a, i.e. chunk 4 vt + vw.
  const int q4 = lane >> 4, ja = lane & 15;
  const int vj = ja >> 2, va = ja & 3;
  const int vrow = tp * TPW + 4 * (q4 >> 1) + vj;
  const int vw = 2 * (q4 & 1) + (va >> 1);
  const int v_off_e = vrow * 1024 + 16 * (vw ^ swz(vrow)) + 8 * (va & 1);
  const int v_off_o = vrow * 1024 + 16 * ((vw + 4) ^ swz(vrow)) + 8 * (va & 1);

  f32x16 acc[VT];
#pragma unroll
  for (int i = 0; i < VT; ++i) acc[i] = f32x16{};
  float m_run = -1e30f, l_run = 0.f;

  for (int blk = 0; blk < nblk; ++blk) {
    wait_stages<C::LPW, C::NS>(min(C::NS - 2, nblk - 1 - blk));
    __syncthreads();  // stage blk visible to all waves; stage blk-1 free
    if (blk + C::NS - 1 < nblk)
      issue_stage<NTP>(kvb, t0 + (blk + C::NS - 1) * C::BT, t1, lds0 + ((blk + C::NS - 1) % C::NS) * C::STAGE_B,
                       wave, lane);
    const unsigned char* st = smem + (blk % C::NS) * C::STAGE_B;

    // ---- S^T (32 tokens x 32 heads) ----
    f32x16 sc = f32x16{};
    {
      u32x4 kf[4];
#pragma unroll
      for (int ks = 0; ks < 3; ++ks) kf[ks] = kread(st, ks);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 3 < KS) kf[(ks + 3) & 3] = kread(st, ks + 3);
        sc = mfma32<BF16>(kf[ks & 3], qf[ks], sc);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // ---- online softmax over this wave's 32 tokens ----
    // lane holds head `head`, tokens tb + 8 i + 4 hsel + j for sc[4 i + j]
    const int tb = t0 + blk * C::BT + tp * TPW;
    const bool need_mask = tb + TPW > t1;
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = sc[r] * sl2;
      if (need_mask && tb + 8 * (r >> 2) + 4 * hsel + (r & 3) >= t1) x = -INFINITY;
      sc[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = max_xor32(mx);
    if (__any(mx > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, mx);
      const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) scale_acc(acc[vt], corr);
    }
    u32x4 pf[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(sc[8 * k2 + e] - m_run);
      pf[k2] = u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                     pack_bf16x2(p[6], p[7])};
#pragma unroll
      for (int w = 0; w < 4; ++w) l_run = dot2_ones<BF16>(pf[k2][w], l_run);
    }

    // ---- O^T += V^T . P^T  (k order: tokens 4 hsel + j, then 8 + 4 hsel + j) ----
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const unsigned char* vb = st + 16 * k2 * 1024;
      auto vread = [&](int vt) {
        const unsigned char* p = vb + ((vt & 1) ? v_off_o : v_off_e) + 128 * (vt >> 1);
        const u32x2 lo = lds_read_tr16(p);
        const u32x2 hi = lds_read_tr16(p + 8 * 1024);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vf[3];
      vf[0] = vread(0);
      vf[1] = vread(1);
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        if (vt + 2 < VT) vf[(vt + 2) % 3] = vread(vt + 2);
        acc[vt] = mfma32<BF16>(vf[vt % 3], pf[k2], acc[vt]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  float l_tot = sum_xor32(l_run);

  if constexpr (NTP > 1) {
    // Merge the token parts of each head group through LDS (the ring is
    // free once every wave is past its last stage).
    static_assert(NTP == 2, "two token parts");
    __syncthreads();
    float* xo = reinterpret_cast<float*>(smem) + hgi * (VT * 16 * 64);
    float* xml = reinterpret_cast<float*>(smem) + C::NHG * VT * 16 * 64 + hgi * 128;
    if (tp == 1) {
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
#pragma unroll
        for (int e = 0; e < 16; ++e) xo[(vt * 16 + e) * 64 + lane] = acc[vt][e];
      xml[lane] = m_run;
      xml[64 + lane] = l_tot;
    }
    __syncthreads();
    if (tp == 1) return;
    const float m_o = xml[lane], l_o = xml[64 + lane];
    const float m_new = fmaxf(m_run, m_o);
    const float ws = __builtin_amdgcn_exp2f(m_run - m_new), wo = __builtin_amdgcn_exp2f(m_o - m_new);
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[vt][e] = acc[vt][e] * ws + xo[(vt * 16 + e) * 64 + lane] * wo;
    l_tot = l_tot * ws + l_o * wo;
    m_run = m_new;
  }

  // lane holds head `head`, dv = 32 vt + 8 i + 4 hsel + j for acc[vt][4 i + j]
  if (nsplit == 1) {
    if (!head_ok) return;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = O + ((size_t)b * H + head) * DV + 4 * hsel;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st64(orow + 32 * vt + 8 * i, u32x2{pack_bf16x2(acc[vt][4 * i] * inv, acc[vt][4 * i + 1] * inv),
                                           pack_bf16x2(acc[vt][4 * i + 2] * inv, acc[vt][4 * i + 3] * inv)});
    return;
  }
  // Partials, lane-major: ws_o[((b * nsplit + s) * HW + hw) * 64 (vt, i) slots][lane] as float4.
  const int HW = (H + HPW - 1) / HPW;
  if (hw >= HW) return;  // a wave whose 32 heads are all padding
  float* po = ws_o + (((size_t)b * nsplit + s) * HW + hw) * (VT * 4 * 64 * 4);
#pragma unroll
  for (int vt = 0; vt < VT; ++vt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<f32x4*>(po + ((vt * 4 + i) * 64 + lane) * 4) =
          f32x4{acc[vt][4 * i], acc[vt][4 * i + 1], acc[vt][4 * i + 2], acc[vt][4 * i + 3]};
  if (hsel == 0) {
    float* pml = ws_ml + (((size_t)b * nsplit + s) * HW + hw) * 64 + 2 * l32;
    *reinterpret_cast<float2*>(pml) = float2{m_run, l_tot};
  }
}

// Merge the per-split softmax states:  o = sum_s w_s o_s / sum_s w_s l_s,
// w_s = 2^(m_s - max_s m_s).  One workgroup per (b, 32-head group); wave w
// merges dv tiles 4w .. 4w+3 in the lane-major partial layout.
__global__ __launch_bounds__(256) void mla_combine_kernel(const float* __restrict__ ws_o,
                                                         const float* __restrict__ ws_ml,
                                                         uint16_t* __restrict__ O, int H, int nsplit) {
  const int HW = (H + HPW - 1) / HPW;
  const int b = blockIdx.x / HW, hw = blockIdx.x % HW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hsel = lane >> 5;
  const int head = hw * HPW + l32;
  float mmax = -1e30f;
  for (int s = 0; s < nsplit; ++s)
    mmax = fmaxf(mmax, ws_ml[(((size_t)b * nsplit + s) * HW + hw) * 64 + 2 * l32]);
  f32x4 o[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) o[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const size_t g = ((size_t)b * nsplit + s) * HW + hw;
    const float2 ml = *reinterpret_cast<const float2*>(ws_ml + g * 64 + 2 * l32);
    const float w = __builtin_amdgcn_exp2f(ml.x - mmax);
    l = fmaf(w, ml.y, l);
    const float* po = ws_o + g * (VT * 4 * 64 * 4) + (size_t)wave * 16 * 64 * 4;
#pragma unroll
    for (int k = 0; k < 16; ++k) o[k] += w * *reinterpret_cast<const f32x4*>(po + (k * 64 + lane) * 4);
  }
  if (head >= H) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = O + ((size_t)b * H + head) * DV + 4 * hsel;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int vt = wave * 4 + k / 4, i = k % 4;
    st64(orow + 32 * vt + 8 * i,
         u32x2{pack_bf16x2(o[k][0] * inv, o[k][1] * inv), pack_bf16x2(o[k][2] * inv, o[k][3] * inv)});
  }
}

// Token parts per head group: two (64-token stages, 64 heads per
// workgroup) when the heads alone give at least two 64-head groups per
// sequence, which halves the split partials; one otherwise.
inline int pick_ntp(int H) { return H >= 128 ? 2 : 1; }

inline size_t workspace_bytes(int B, int H, int T) {
  const Split sp = pick_ntp(H) == 2 ? pick_split<2>(B, H, T) : pick_split<1>(B, H, T);
  if (sp.nsplit <= 1) return 0;
  const size_t HW = (size_t)(H + HPW - 1) / HPW;
  return (size_t)B * sp.nsplit * HW * (HPW * DV + 2 * HPW) * sizeof(float);
}

template <int NTP>
static int launch(const void* Q, const void* KV, void* O, int B, int H, int T, float sl2, void* workspace,
                  hipStream_t s) {
  using C = Cfg<NTP>;
  const Split sp = pick_split<NTP>(B, H, T);
  const int HGB = (H + C::HPG - 1) / C::HPG;
  const long long grid = (long long)B * HGB * sp.nsplit;
  if (grid > 0x7fffffffLL) return MX_ERR_SHAPE;
  const size_t HW = (size_t)(H + HPW - 1) / HPW;
  float* ws_o = (float*)workspace;
  float* ws_ml = sp.nsplit > 1 ? ws_o + (size_t)B * sp.nsplit * HW * HPW * DV : nullptr;
  MX_RETURN_IF_HIP(hipFuncSetAttribute((const void*)mla_decode_kernel<NTP>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES));
  hipLaunchKernelGGL(mla_decode_kernel<NTP>, dim3((unsigned)grid), dim3(NT), LDS_BYTES, s, (const uint16_t*)Q,
                     (const uint16_t*)KV, (uint16_t*)O, ws_o, ws_ml, B, H, T, sl2, sp.nsplit, sp.tps);
  MX_RETURN_IF_HIP(hipGetLastError());
  if (sp.nsplit > 1) {
    hipLaunchKernelGGL(mla_combine_kernel, dim3((unsigned)(B * HW)), dim3(256), 0, s, ws_o, ws_ml, (uint16_t*)O, H,
                       sp.nsplit);
    MX_RETURN_IF_HIP(hipGetLastError());
  }
  return MX_OK;
}

}  // namespace mla
}  // namespace mx

extern "C" size_t mx_mla_decode_workspace(int B, int H, int T, int d_latent) {
  if (B <= 0 || H <= 0 || T <= 0 || d_latent != mx::mla::DV) return 0;
  return mx::mla::workspace_bytes(B, H, T);
}

extern "C" int mx_mla_decode(const void* Q, const void* KV, void* O, int B, int H, int T, int d_latent, int d_rope,
                             float scale, void* workspace, size_t ws_bytes, void* stream) {
  using namespace mx::mla;
  if (!Q || !KV || !O) return MX_ERR_NULL;
  if (B <= 0 || H <= 0 || T <= 0) return MX_ERR_SHAPE;
  if (d_latent != DV || d_rope != DQK - DV) return MX_ERR_UNSUPPORTED;
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return MX_ERR_SHAPE;
  if ((long long)B * T * DQK > (1LL << 40) || (long long)B * H > (1LL << 30)) return MX_ERR_SHAPE;
  if (((uintptr_t)Q | (uintptr_t)KV | (uintptr_t)O) & 15) return MX_ERR_ALIGN;
  const size_t need = workspace_bytes(B, H, T);
  if (need > 0 && (!workspace || ws_bytes < need)) return MX_ERR_WORKSPACE;
  if (need > 0 && ((uintptr_t)workspace & 15)) return MX_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  if (pick_ntp(H) == 2) return launch<2>(Q, KV, O, B, H, T, sl2, workspace, s);
  return launch<1>(Q, KV, O, B, H, T, sl2, workspace, s);
}
